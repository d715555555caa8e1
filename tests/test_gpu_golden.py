"""GPU: the HIP expert path on the committed tiny-layer fixture. The stored MXFP4 codes
are laid out as tile images on the host, the layer runs through afd_moe_ffn, and the
result must match the stored oracle output within rel-L2 1e-2 with the routing bit-exact.
Re-packing the dequantized fixture weights on the GPU must give the same images (MX
quantization is idempotent on already-quantized values)."""

import numpy as np
import pytest
import torch

import layouts as L
from gpu_util import bits16, dev, rel_l2, say, u8
from oracle import formats as F
from sgl_asap_amd.moe.experts import AfdExperts, ExpertWeights, pack_mxfp4_experts
from sgl_asap_amd.moe.topk import StandardTopKOutput
from test_golden import load

pytestmark = pytest.mark.gpu


def gate_up_rows(rows, g=32):
    """Logical row of each physical row of the gate/up interleave of W13."""
    half = rows // 2
    j, q = np.divmod(np.arange(rows), 2 * g)
    return np.where(q < g, j * g + q, half + j * g + q - g)


def fixture_weights(g):
    h, inter, _, e, _, _ = g["shape"].tolist()
    perm = gate_up_rows(2 * inter)
    img13 = L.b_images(g["w13_packed"][:, perm], g["w13_scales"][:, perm]).reshape(e, -1)
    img2 = L.b_images(g["w2_packed"], g["w2_scales"]).reshape(e, -1)
    none = torch.empty(0, dtype=torch.uint8, device=dev())
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev())
    return ExpertWeights("mxfp4", e, h, inter, to(img13), none, to(img2), none), img13, img2


def test_hip_path_on_fixture():
    say("golden tiny layer through afd_moe_ffn")
    g = load()
    h, inter, ne, e, k, n = g["shape"].tolist()
    weights, _, _ = fixture_weights(g)
    experts = AfdExperts(ne, k, 0, range(0, e), weights, n_max=n)
    x = torch.from_numpy(g["x_bits"].view(np.int16)).view(torch.bfloat16).to(dev())
    topk = StandardTopKOutput(torch.from_numpy(g["topk_weights"]).to(dev()), torch.from_numpy(g["topk_ids"]).to(dev()))
    out = experts(x, topk)
    torch.cuda.synchronize()
    for key, dtype in (("counts", torch.int32), ("padded_offsets", torch.int32), ("sorted_pairs", torch.int32), ("pair_pos", torch.int32)):
        got = experts.ws_view(key, dtype, g[key].size, n).cpu().numpy()
        assert np.array_equal(got, g[key]), key
    err = rel_l2(F.bf16_to_f32(bits16(out)), F.bf16_to_f32(g["out_bits"]))
    say(f"rel_l2={err:.3e}")
    assert err <= 1e-2


def test_gpu_pack_is_idempotent_on_fixture_codes():
    say("golden tiny layer: GPU pack of the dequantized codes")
    g = load()
    _, img13, img2 = fixture_weights(g)
    w13 = F.mx_dequantize(F.unpack_fp4(g["w13_packed"]), g["w13_scales"], "e2m1")
    w2 = F.mx_dequantize(F.unpack_fp4(g["w2_packed"]), g["w2_scales"], "e2m1")
    packed = pack_mxfp4_experts(torch.from_numpy(w13), torch.from_numpy(w2), device=dev())
    torch.cuda.synchronize()
    assert np.array_equal(u8(packed.w13), img13)
    assert np.array_equal(u8(packed.w2), img2)
