"""Number formats of the expert path, restated bit by bit in numpy (test infrastructure).

The reference hands these formats to third-party kernels (SGLang / FlashInfer MXFP4,
``python/sgl_asap_plugin/srt/layers/quantization/mxfp4_flashinfer_trtllm_moe.py:49-61``;
checkpoint format ``python/sgl_asap_plugin/srt/configs/model_config.py:3-7``: int8-packed
e2m1 + E8M0 per 32). Their exact rounding is not in the reference tree, so the build
defines it from the OCP MX v1.0 and OCP FP8 specifications:

* E2M1 (fp4): magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6}, sign in bit 3; element 2i of a
  row sits in the low nibble of byte i. Round to nearest, ties to even code; saturate at 6.
* UE8M0 scale: value 2^(code - 127); 255 is NaN.
* e4m3fn (OCP, gfx950's FP8): bias 7, max 448, subnormals down to 2^-9, 0x7F/0xFF NaN.
  Round to nearest even.
* MX block of 32 along K: shared exponent floor(log2(amax)) - emax_elem (emax 2 for E2M1,
  8 for e4m3), clamped to [-127, 127]; amax == 0 gives code 0. Elements are
  v * 2^-(shared exponent), rounded, saturated.
* FP8 block (1x128 activations, 128x128 weights): s = max(amax, 1e-10) / 448 in fp32;
  q = e4m3(clamp(v / s, -448, 448)).

Pinned by: exhaustive decode tables against torch's float8_e4m3fn / float8_e8m0fnu casts;
the e4m3 encoder against torch's RNE cast on dense sweeps; E2M1 against the OCP value table
and its tie cases; quantize/dequantize round-trip bounds.
"""

from __future__ import annotations

import numpy as np

E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
E4M3_MAX = 448.0
MX_BLOCK = 32
FP8_BLOCK = 128
FP8_EPS = 1e-10


def _f32_bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> fp32 values (exact)."""
    return (np.asarray(u16, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even; NaN stays a quiet NaN.
    Same rounding as torch's ``.to(torch.bfloat16)``."""
    u = _f32_bits(a).astype(np.uint64)
    nan = np.isnan(np.asarray(a, dtype=np.float32))
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = (rounded & 0xFFFF).astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


# ---------------------------------------------------------------- E2M1 (fp4)
def e2m1_decode(codes: np.ndarray) -> np.ndarray:
    """4-bit codes (0..15) -> fp32."""
    c = np.asarray(codes, dtype=np.uint8)
    mag = E2M1_VALUES[c & 7]
    return np.where(c & 8, -mag, mag).astype(np.float32)


def e2m1_encode(v: np.ndarray) -> np.ndarray:
    """fp32 (already divided by the block scale) -> 4-bit codes, RNE, saturating at 6.
    The tie points 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5 go to the even code."""
    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v)
    code = (
        (a > 0.25).astype(np.uint8)
        + (a >= 0.75)
        + (a > 1.25)
        + (a >= 1.75)
        + (a > 2.5)
        + (a >= 3.5)
        + (a > 5.0)
    ).astype(np.uint8)
    sign = (_f32_bits(v) >> 31).astype(np.uint8)
    return code | (sign << 3)


def pack_fp4(codes: np.ndarray) -> np.ndarray:
    """[..., K] 4-bit codes -> [..., K/2] bytes, element 2i in the low nibble."""
    c = np.asarray(codes, dtype=np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def unpack_fp4(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


# ---------------------------------------------------------------- UE8M0
def ue8m0_decode(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.int32)
    with np.errstate(over="ignore"):
        val = np.ldexp(np.float32(1.0), c - 127).astype(np.float32)
    return np.where(c == 255, np.float32(np.nan), val).astype(np.float32)


# ---------------------------------------------------------------- e4m3fn
def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.int32)
    s = c >> 7
    e = (c >> 3) & 15
    m = c & 7
    sub = np.ldexp(m.astype(np.float64), -9)
    nrm = np.ldexp(1.0 + m / 8.0, e - 7)
    mag = np.where(e == 0, sub, nrm)
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(s == 1, -mag, mag).astype(np.float32)


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """fp32 with |v| <= 448 (callers clamp first) -> e4m3fn codes, RNE. Bit-level:
    normals keep 3 mantissa bits of the fp32 significand with ties to even; below 2^-6
    the value is rint(|v| * 2^9) subnormal steps (8 steps = the smallest normal)."""
    v = np.asarray(v, dtype=np.float32)
    u = _f32_bits(v).astype(np.int64)
    sign = (u >> 31) & 1
    mag_bits = u & 0x7FFFFFFF
    exp32 = mag_bits >> 23
    man = mag_bits & 0x7FFFFF
    e = exp32 - 127
    keep = man >> 20
    rem = man & 0xFFFFF
    up = (rem > 0x80000) | ((rem == 0x80000) & ((keep & 1) == 1))
    m = keep + up
    e_n = e + (m >> 3)
    m = m & 7
    normal_code = ((e_n + 7) << 3) | m
    a = np.abs(v).astype(np.float32)
    sub_code = np.rint(a * np.float32(512.0)).astype(np.int64)  # exact product, RNE
    code = np.where(e >= -6, normal_code, sub_code)
    return (code | (sign << 7)).astype(np.uint8)


# ---------------------------------------------------------------- MX block quantizers
def _mx_scale_codes(amax: np.ndarray, emax: int) -> np.ndarray:
    exp32 = ((_f32_bits(amax) >> 23) & 0xFF).astype(np.int64)
    e = np.where(exp32 > 0, exp32 - 127, -127)
    code = np.clip(e - emax + 127, 0, 254)
    return np.where(amax == 0, 0, code).astype(np.uint8)


def _pow2_neg(codes: np.ndarray) -> np.ndarray:
    """2^(127 - code) as fp32 (exact for code in [0, 253])."""
    return np.ldexp(np.float32(1.0), 127 - codes.astype(np.int32)).astype(np.float32)


def mx_quantize(v: np.ndarray, elem: str):
    """Row-wise MX quantization along the last axis in blocks of 32.

    v: fp32 [..., K], K % 32 == 0. elem: "e2m1" or "e4m3".
    Returns (codes uint8 [..., K] (unpacked for e2m1), scales uint8 [..., K/32]).
    """
    v = np.asarray(v, dtype=np.float32)
    k = v.shape[-1]
    assert k % MX_BLOCK == 0, k
    blocks = v.reshape(v.shape[:-1] + (k // MX_BLOCK, MX_BLOCK))
    amax = np.max(np.abs(blocks), axis=-1)
    emax = 2 if elem == "e2m1" else 8
    scales = _mx_scale_codes(amax, emax)
    scaled = blocks * _pow2_neg(scales)[..., None]
    if elem == "e2m1":
        codes = e2m1_encode(scaled)
    else:
        codes = e4m3_encode(np.clip(scaled, -E4M3_MAX, E4M3_MAX))
    return codes.reshape(v.shape), scales


def mx_dequantize(codes: np.ndarray, scales: np.ndarray, elem: str) -> np.ndarray:
    codes = np.asarray(codes, dtype=np.uint8)
    k = codes.shape[-1]
    vals = e2m1_decode(codes) if elem == "e2m1" else e4m3_decode(codes)
    vals = vals.reshape(codes.shape[:-1] + (k // MX_BLOCK, MX_BLOCK))
    return (vals * ue8m0_decode(scales)[..., None]).reshape(codes.shape).astype(np.float32)


# ---------------------------------------------------------------- FP8 block quantizers
def fp8_group_quantize(v: np.ndarray, group: int = FP8_BLOCK):
    """Per-row groups of ``group`` along the last axis (activations, 1x128):
    s = max(amax, 1e-10) / 448, q = e4m3(clamp(v / s)). -> (codes [.., K], s fp32 [.., K/group])."""
    v = np.asarray(v, dtype=np.float32)
    k = v.shape[-1]
    b = v.reshape(v.shape[:-1] + (k // group, group))
    amax = np.max(np.abs(b), axis=-1)
    s = (np.maximum(amax, np.float32(FP8_EPS)) / np.float32(E4M3_MAX)).astype(np.float32)
    q = np.clip(b / s[..., None], -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return e4m3_encode(q).reshape(v.shape), s


def fp8_block_quantize_2d(w: np.ndarray, block: int = FP8_BLOCK):
    """[..., N, K] weights in 128x128 blocks -> (codes [..., N, K], s fp32 [..., N/128, K/128])."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape[-2:]
    lead = w.shape[:-2]
    b = w.reshape(lead + (n // block, block, k // block, block))
    amax = np.max(np.abs(b), axis=(-3, -1))
    s = (np.maximum(amax, np.float32(FP8_EPS)) / np.float32(E4M3_MAX)).astype(np.float32)
    q = np.clip(b / s[..., :, None, :, None], -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return e4m3_encode(q).reshape(w.shape), s


def fp8_group_dequantize(codes: np.ndarray, s: np.ndarray, group: int = FP8_BLOCK) -> np.ndarray:
    vals = e4m3_decode(codes)
    k = vals.shape[-1]
    vals = vals.reshape(vals.shape[:-1] + (k // group, group)) * s[..., None]
    return vals.reshape(codes.shape).astype(np.float32)


def fp8_block_dequantize_2d(codes: np.ndarray, s: np.ndarray, block: int = FP8_BLOCK) -> np.ndarray:
    vals = e4m3_decode(codes)
    n, k = vals.shape[-2:]
    lead = vals.shape[:-2]
    b = vals.reshape(lead + (n // block, block, k // block, block)) * s[..., :, None, :, None]
    return b.reshape(vals.shape).astype(np.float32)
