"""Pins the oracle's number formats (CPU): decoders against torch's float8 casts and the
E2M1 bit-field formula, encoders against torch's round-to-nearest-even cast and a
brute-force nearest-value search, MX scale choice against frexp, quantizer round-trip
bounds, and the fp4 nibble order against the checkpoint convention."""

import math

import numpy as np
import pytest
import torch

from oracle import formats as F


def all_e4m3_values():
    c = np.arange(256, dtype=np.uint8)
    v = torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy()
    return c, v


def test_e4m3_decode_matches_torch_all_codes():
    c, want = all_e4m3_values()
    got = F.e4m3_decode(c)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan) and nan.sum() == 2  # 0x7F and 0xFF
    assert np.array_equal(got[~nan], want[~nan])
    assert F.e4m3_decode(np.array([0x7E]))[0] == 448.0


def test_ue8m0_decode_matches_torch_all_codes():
    c = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(c).view(torch.float8_e8m0fnu).float().numpy()
    got = F.ue8m0_decode(c)
    assert np.isnan(got[255]) and np.isnan(want[255])
    assert np.array_equal(got[:255], want[:255])


def test_e2m1_decode_from_bit_fields():
    """E2M1: sign bit 3, exponent bits 2-1 (bias 1), mantissa bit 0; e == 0 is subnormal."""
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        assert F.e2m1_decode(np.array([code]))[0] == (-mag if s else mag)


def _e4m3_sweep():
    _, vals = all_e4m3_values()
    finite = np.unique(vals[np.isfinite(vals) & (vals >= 0)]).astype(np.float64)
    mids = (finite[:-1] + finite[1:]) / 2  # exact in fp32: the tie points
    pts = np.concatenate([finite, mids]).astype(np.float32)
    nb = np.concatenate([pts, np.nextafter(pts, np.float32(0)), np.nextafter(pts, np.float32(1e4))])
    rng = np.random.default_rng(0)
    rnd = np.concatenate([
        rng.uniform(-448, 448, 200_000),
        np.exp(rng.uniform(math.log(1e-6), math.log(448), 200_000)),
    ]).astype(np.float32)
    v = np.concatenate([nb, -nb, rnd, -rnd]).astype(np.float32)
    return v[np.abs(v) <= 448]


def test_e4m3_encode_matches_torch_rne_cast():
    v = _e4m3_sweep()
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = F.e4m3_encode(v)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (v[bad[:5]], got[bad[:5]], want[bad[:5]])


def test_e2m1_encode_is_nearest_value_ties_to_even_code():
    """Brute force: the code whose value is nearest; on a tie, the even code; above 6, 6."""
    grid = np.concatenate([np.arange(0, 7.0, 0.03125), [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.5, 100.0]])
    v = np.concatenate([grid, -grid]).astype(np.float32)
    got = F.e2m1_encode(v)
    for x, code in zip(v.tolist(), got.tolist()):
        d = [abs(abs(x) - F.E2M1_VALUES[c]) for c in range(8)]
        best = min(d)
        cands = [c for c in range(8) if d[c] == best]
        want = cands[0] if len(cands) == 1 else [c for c in cands if c % 2 == 0][0]
        sign = 8 if math.copysign(1.0, x) < 0 else 0
        assert code == want | sign, (x, code, want)


def test_fp4_nibble_order():
    """Element 2i in the low nibble of byte i (the int8-packed e2m1 checkpoint format)."""
    assert F.pack_fp4(np.array([1, 2, 3, 4, 15, 0], dtype=np.uint8)).tolist() == [0x21, 0x43, 0x0F]
    codes = np.random.default_rng(1).integers(0, 16, (3, 64), dtype=np.uint8)
    assert np.array_equal(F.unpack_fp4(F.pack_fp4(codes)), codes)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 1 << 32, 300_000, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    ties = (rng.integers(0, 1 << 16, 1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    v = np.concatenate([v, ties, np.array([np.inf, -np.inf, 0.0, -0.0], dtype=np.float32)])
    v = v[~np.isnan(v)]
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(F.f32_to_bf16(v), want)
    assert np.isnan(F.bf16_to_f32(F.f32_to_bf16(np.array([np.nan], dtype=np.float32))))[0]


@pytest.mark.parametrize("elem,emax", [("e2m1", 2), ("e4m3", 8)])
def test_mx_scale_is_floor_log2_amax_minus_emax(elem, emax):
    rng = np.random.default_rng(3)
    amax = np.exp(rng.uniform(math.log(1e-30), math.log(1e30), 5000)).astype(np.float32)
    amax = np.concatenate([amax, np.float32([1.0, 2.0, 4.0, 0.75, 6.0, 448.0, 2.0 ** -126, 1e-45])])
    blocks = np.zeros((amax.size, 32), dtype=np.float32)
    blocks[:, 7] = -amax  # amax is an absolute value
    blocks[:, 3] = amax / 3
    _, scales = F.mx_quantize(blocks, elem)
    for a, s in zip(amax.tolist(), scales[:, 0].tolist()):
        m, e = math.frexp(a)  # a = m * 2^e, m in [0.5, 1)
        want = min(max((e - 1) - emax + 127, 0), 254)
        assert s == want, (a, s, want)
    zero_codes, zero_scales = F.mx_quantize(np.zeros((2, 64), dtype=np.float32), elem)
    assert not zero_codes.any() and not zero_scales.any()


@pytest.mark.parametrize("elem", ["e2m1", "e4m3"])
def test_mx_round_trip_bounds(elem):
    rng = np.random.default_rng(4)
    v = (rng.standard_normal((64, 256)) * np.exp(rng.uniform(-8, 8, (64, 1)))).astype(np.float32)
    codes, scales = F.mx_quantize(v, elem)
    back = F.mx_dequantize(codes, scales, elem)
    x = F.ue8m0_decode(scales).repeat(32, axis=1)
    if elem == "e2m1":  # step 2 between 4 and 6 (err <= X), saturation of (6X, 8X) (err < 2X)
        assert np.all(np.abs(back - v) <= 2 * x)
    else:  # 3 mantissa bits: half a step is 2^-4 of the value; (448 X, 512 X) saturates to 448 X
        sat = np.abs(v) > 448 * x
        ok = np.abs(back - v) <= np.maximum(np.abs(v) * 2.0 ** -4, x * 2.0 ** -9) + 1e-30
        assert np.all(ok[~sat]) and sat.any()
        assert np.array_equal(np.abs(back[sat]), 448 * x[sat])
        assert np.all(np.abs(v) / x < 512)
    # the block maximum lands in the format's top binade
    top = np.abs(back).reshape(64, 8, 32).max(-1) / F.ue8m0_decode(scales)
    lo = 4.0 if elem == "e2m1" else 256.0
    assert np.all(top >= lo)


def test_fp8_group_quantizer_scale_and_codes():
    rng = np.random.default_rng(5)
    v = (rng.standard_normal((8, 512)) * 3).astype(np.float32)
    v[1, :128] = 0.0  # an all-zero group: scale 1e-10 / 448, codes 0
    codes, s = F.fp8_group_quantize(v)
    tv = torch.from_numpy(v).view(8, 4, 128)
    want_s = (tv.abs().amax(-1).clamp_min(1e-10) / 448.0).numpy()
    assert np.array_equal(s, want_s)
    want = (tv / torch.from_numpy(s)[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert np.array_equal(codes, want.view(torch.uint8).reshape(8, 512).numpy())
    assert not codes[1, :128].any()
    back = F.fp8_group_dequantize(codes, s)
    half_sub = np.repeat(s, 128, axis=1) * 2.0 ** -10  # half a subnormal step
    assert np.all(np.abs(back - v) <= np.maximum(np.abs(v) * 2.0 ** -4, half_sub))


def test_fp8_block_2d_uses_the_128x128_block_maximum():
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((2, 256, 384)) * 0.02).astype(np.float32)
    w[1, 130, 5] = 7.0  # one outlier scales exactly one block
    codes, s = F.fp8_block_quantize_2d(w)
    assert s.shape == (2, 2, 3)
    for e in range(2):
        for i in range(2):
            for j in range(3):
                blk = w[e, i * 128:(i + 1) * 128, j * 128:(j + 1) * 128]
                assert s[e, i, j] == np.float32(max(np.abs(blk).max(), 1e-10)) / np.float32(448)
    assert s[1, 1, 0] == np.float32(7.0) / np.float32(448) and codes[1, 130, 5] == 0x7E
    back = F.fp8_block_dequantize_2d(codes, s)
    assert np.all(np.abs(back - w) <= np.abs(w) * 2.0 ** -4 + s.max() * 2.0 ** -9)
