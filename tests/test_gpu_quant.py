"""GPU parity: the HIP quantizers and weight packers are bit-exact with the oracle."""

import numpy as np
import pytest
import torch

import layouts as L
from gpu_util import dev, say, u8
from oracle import formats as F
from sgl_asap_amd import _lib

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _e4m3_ties():
    """Every positive e4m3 midpoint (normal and subnormal), its bf16 neighbours and the
    negatives: values that the quantizers see unchanged when the group's scale is 1."""
    vals = np.array([float(F.e4m3_decode(np.array([c], dtype=np.uint8))[0]) for c in range(127)])
    mids = (vals[:-1] + vals[1:]) / 2
    bf = torch.tensor(mids, dtype=torch.float32).to(torch.bfloat16)
    up = (bf.view(torch.int16) + 1).view(torch.bfloat16)
    down = (bf.view(torch.int16) - 1).view(torch.bfloat16)
    pos = torch.cat([bf, up, down]).float()
    return torch.cat([pos, -pos])


def _tie_row(cols, group, amax):
    """A row whose every `group` elements start with `amax` (scale exactly 1: 448 for FP8
    1x128, 256 for MXFP8) followed by e4m3 ties."""
    ties = _e4m3_ties()
    row = torch.empty(cols)
    k = 0
    for g0 in range(0, cols, group):
        row[g0] = amax
        for c in range(g0 + 1, g0 + group):
            row[c] = ties[k % len(ties)]
            k += 1
    return row


def _bf16_input(rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * torch.logspace(-3, 3, cols)[None, :]
    if rows >= 3:
        x[0, :] = 0.0  # an all-zero row: scale code 0
        x[1, :32] = 1e-30  # a tiny block
        x[2, :64] = torch.tensor([0.25, -0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 448.0] * 8)
    if rows >= 5 and cols >= 128:
        x[3] = _tie_row(cols, 128, 448.0)  # FP8 1x128 groups with scale 1: RNE ties
        x[4] = _tie_row(cols, 32, 256.0)  # MXFP8 blocks with scale 2^0
    return x.to(torch.bfloat16)


def _x_f32(x):
    return F.bf16_to_f32(x.contiguous().view(torch.int16).numpy().view(np.uint16))


@pytest.mark.parametrize("rows,cols", [(1, 32), (37, 512), (129, 4096)])
def test_quant_mxfp8_bitexact(rows, cols):
    say(f"quant_mxfp8 rows={rows} cols={cols}")
    x = _bf16_input(rows, cols, seed=rows)
    xd = x.to(dev())
    q = torch.empty(rows, cols, dtype=torch.uint8, device=dev())
    s = torch.empty(rows, cols // 32, dtype=torch.uint8, device=dev())
    _lib.call("afd_quant_mxfp8", xd.data_ptr(), rows, cols, q.data_ptr(), s.data_ptr(), _stream())
    torch.cuda.synchronize()
    q_ref, s_ref = F.mx_quantize(_x_f32(x), "e4m3")
    assert np.array_equal(u8(s), s_ref)
    assert np.array_equal(u8(q), q_ref)


@pytest.mark.parametrize("rows,cols", [(1, 128), (37, 512), (129, 4096)])
def test_quant_fp8_1x128_bitexact(rows, cols):
    say(f"quant_fp8_1x128 rows={rows} cols={cols}")
    x = _bf16_input(rows, cols, seed=rows + 7)
    xd = x.to(dev())
    q = torch.empty(rows, cols, dtype=torch.uint8, device=dev())
    s = torch.empty(rows, cols // 128, dtype=torch.float32, device=dev())
    _lib.call("afd_quant_fp8_1x128", xd.data_ptr(), rows, cols, q.data_ptr(), s.data_ptr(), _stream())
    torch.cuda.synchronize()
    q_ref, s_ref = F.fp8_group_quantize(_x_f32(x))
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(u8(q), q_ref)


def _gate_up_rows(rows, g=32):
    """Logical row of each physical row of the gate/up interleave."""
    half = rows // 2
    out = []
    for r in range(rows):
        j, q = divmod(r, 2 * g)
        out.append(j * g + q if q < g else half + j * g + q - g)
    return np.array(out)


@pytest.mark.parametrize("gate_up", [0, 1])
def test_pack_mxfp4_bitexact(gate_up):
    say(f"pack_mxfp4 gate_up={gate_up}")
    g = torch.Generator().manual_seed(3)
    mats, rows, cols = 3, 512, 384
    w = torch.randn(mats, rows, cols, generator=g) * 0.02
    w[0, 0, :32] = 0.0
    w[1, 5, :8] = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0])
    wd = w.to(dev())
    out = torch.empty(mats * rows * (cols // 2 + cols // 32), dtype=torch.uint8, device=dev())
    _lib.call("afd_pack_mxfp4", wd.data_ptr(), mats, rows, cols, gate_up, out.data_ptr(), _stream())
    torch.cuda.synchronize()
    codes, scales = F.mx_quantize(w.numpy(), "e2m1")
    packed = F.pack_fp4(codes)
    if gate_up:
        perm = _gate_up_rows(rows)
        packed, scales = packed[:, perm], scales[:, perm]
    assert np.array_equal(u8(out), L.b_images(packed, scales).reshape(-1))


@pytest.mark.parametrize("gate_up", [0, 1])
def test_pack_fp8_block_bitexact(gate_up):
    say(f"pack_fp8_block gate_up={gate_up}")
    g = torch.Generator().manual_seed(4)
    mats, rows, cols = 2, 256, 384
    w = torch.randn(mats, rows, cols, generator=g) * 0.02
    wd = w.to(dev())
    q = torch.empty(mats, rows, cols, dtype=torch.uint8, device=dev())
    s = torch.empty(mats, rows // 128, cols // 128, dtype=torch.float32, device=dev())
    _lib.call("afd_pack_fp8_block", wd.data_ptr(), mats, rows, cols, gate_up, q.data_ptr(), s.data_ptr(), _stream())
    torch.cuda.synchronize()
    codes, scales = F.fp8_block_quantize_2d(w.numpy())
    if gate_up:
        codes = codes[:, _gate_up_rows(rows)]
    assert np.array_equal(s.cpu().numpy().view(np.uint32), scales.view(np.uint32))
    assert np.array_equal(u8(q).reshape(-1), L.fp8_images(codes).reshape(-1))
