"""GPU: the checkpoint repack kernels move a quantized checkpoint's bytes into the kernel's
layouts unchanged (bit-exact against the numpy statement of the layouts), and a layer loaded
from a synthetic safetensors checkpoint computes what the oracle computes with the
checkpoint's dequantized weights."""

import numpy as np
import pytest
import torch

import ckpt
import layouts as L
from gpu_util import bits16, dev, rel_l2, say, u8
from oracle import experts as OX
from oracle import formats as F
from sgl_asap_amd import _lib
from sgl_asap_amd import workloads as W
from sgl_asap_amd.loader import load_routed_experts
from sgl_asap_amd.moe.experts import AfdExperts, pack_mxfp4_experts
from sgl_asap_amd.moe.topk import StandardTopKOutput

pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-2


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _gate_up_rows(rows, g=32):
    half = rows // 2
    out = []
    for r in range(rows):
        j, q = divmod(r, 2 * g)
        out.append(j * g + q if q < g else half + j * g + q - g)
    return np.array(out)


@pytest.mark.parametrize("gate_up", [0, 1])
def test_repack_mxfp4_bitexact(gate_up):
    say(f"repack_mxfp4 gate_up={gate_up}")
    g = np.random.default_rng(7)
    mats, rows, cols = 3, 512, 384
    codes, scales = F.mx_quantize((g.standard_normal((mats, rows, cols)) * 0.02).astype(np.float32), "e2m1")
    packed = F.pack_fp4(codes)
    out = torch.empty(mats * rows * (cols // 2 + cols // 32), dtype=torch.uint8, device=dev())
    pd, sd = torch.from_numpy(packed).to(dev()), torch.from_numpy(scales).to(dev())
    _lib.call("afd_repack_mxfp4", pd.data_ptr(), sd.data_ptr(), mats, rows, cols, gate_up, out.data_ptr(), _stream())
    torch.cuda.synchronize()
    if gate_up:
        perm = _gate_up_rows(rows)
        packed, scales = packed[:, perm], scales[:, perm]
    assert np.array_equal(u8(out), L.b_images(packed, scales).reshape(-1))


@pytest.mark.parametrize("gate_up", [0, 1])
def test_repack_fp8_block_bitexact(gate_up):
    say(f"repack_fp8_block gate_up={gate_up}")
    g = np.random.default_rng(8)
    mats, rows, cols = 2, 256, 384
    codes, _ = F.fp8_block_quantize_2d((g.standard_normal((mats, rows, cols)) * 0.02).astype(np.float32))
    qd = torch.from_numpy(codes).to(dev())
    out = torch.empty_like(qd)
    _lib.call("afd_repack_fp8_block", qd.data_ptr(), mats, rows, cols, gate_up, out.data_ptr(), _stream())
    torch.cuda.synchronize()
    rows_in_order = codes[:, _gate_up_rows(rows)] if gate_up else codes
    assert np.array_equal(u8(out).reshape(-1), L.fp8_images(rows_in_order).reshape(-1))


def test_repack_rejects_bad_shapes_and_alignment():
    say("repack argument checks")
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device=dev())
    p = buf.data_ptr()
    with pytest.raises(ValueError):
        _lib.call("afd_repack_mxfp4", p, p, 1, 300, 256, 0, p, _stream())  # rows % 256
    with pytest.raises(ValueError):
        _lib.call("afd_repack_mxfp4", p + 1, p, 1, 256, 256, 0, p, _stream())  # misaligned codes
    with pytest.raises(ValueError):
        _lib.call("afd_repack_fp8_block", p, 1, 128, 256, 1, p, _stream())  # gate_up rows % 256


@pytest.mark.parametrize("fmt,naming", [("mxfp4", "dsv4"), ("mxfp4", "hf"), ("fp8_block", "hf"), ("fp8_block", "dsv4")])
def test_layer_from_checkpoint_matches_oracle(tmp_path, fmt, naming):
    say(f"checkpoint load {fmt} {naming}")
    H, I, E, K, n = 256, 128, 12, 4, 96
    local = range(4, 10)
    files, logical = ckpt.write_checkpoint(str(tmp_path), layers=2, num_experts=E, hidden=H, inter=I,
                                           fmt=fmt, naming=naming, seed=3)
    weights = load_routed_experts(files, local, num_layers=2, device=dev())
    assert sorted(weights) == [0, 1]
    gen = W.generator("cpu", 11)
    x = W.tokens(n, H, gen, "cpu")
    ids, w = W.route_uniform(n, E, K, gen, "cpu")
    act = "mxfp8" if fmt == "mxfp4" else "fp8_1x128"
    for layer, ew in weights.items():
        assert ew.fmt == fmt and (ew.num_local, ew.hidden, ew.inter) == (len(local), H, I)
        experts = AfdExperts(E, K, layer, local, ew, n_max=n)
        out = experts(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev())))
        torch.cuda.synchronize()
        w13, w2 = (a[local.start:local.stop] for a in logical[layer])
        ref = OX.moe_ffn(x, ids.numpy(), w.numpy(), ckpt.dequantized(w13, fmt), ckpt.dequantized(w2, fmt),
                         local.start, act=act)
        err = rel_l2(F.bf16_to_f32(bits16(out)), F.bf16_to_f32(ref))
        assert err <= REL_L2_TOL, (layer, err)
        if fmt == "mxfp4":
            # an MX block's largest element quantizes to 4 or 6 at its scale, so the dequantized
            # checkpoint requantizes to the same codes and scales: packing those weights gives
            # the repacked images byte for byte
            packed = pack_mxfp4_experts(torch.from_numpy(ckpt.dequantized(w13, fmt)),
                                        torch.from_numpy(ckpt.dequantized(w2, fmt)), device=dev())
            torch.cuda.synchronize()
            assert torch.equal(packed.w13, ew.w13) and torch.equal(packed.w2, ew.w2)
