"""Pins the oracle's expert call, finalize and combine (CPU): a float64 per-token dense
MLP written independently of the oracle's routed formulation, exact special cases (no
local pair, zero weights, repeated tokens, power-of-two weight scaling), and the
finalize / combine formulas against torch fp32 arithmetic, bit for bit."""

import math

import numpy as np
import pytest
import torch

from oracle import experts as OX
from oracle import formats as F

H, I = 256, 128


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def setup(n, k, num_experts, e_lo, num_local, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, H, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(num_experts, generator=g)[:k] for _ in range(n)]).to(torch.int32)
    w = torch.rand(n, k, generator=g)
    w13 = (torch.randn(num_local, 2 * I, H, generator=g) * 0.05).numpy()
    w2 = (torch.randn(num_local, H, I, generator=g) * 0.05).numpy()
    return x, ids.numpy(), w.numpy(), w13, w2


def dense_reference(x, ids, w, w13, w2, e_lo):
    """float64, token by token: sum over local picks of w * bf16(W2 . bf16(silu(Wg x) * (Wu x)))."""
    xf = x.double().numpy()
    n, k = ids.shape
    out = np.zeros((n, H))
    for t in range(n):
        for kk in range(k):
            e = int(ids[t, kk]) - e_lo
            if not 0 <= e < w13.shape[0]:
                continue
            wg, wu = w13[e, :I].astype(np.float64), w13[e, I:].astype(np.float64)
            g, u = wg @ xf[t], wu @ xf[t]
            h = g / (1 + np.exp(-g)) * u
            h = F.bf16_to_f32(F.f32_to_bf16(h.astype(np.float32))).astype(np.float64)
            y = F.bf16_to_f32(F.f32_to_bf16((w2[e].astype(np.float64) @ h).astype(np.float32)))
            out[t] += float(w[t, kk]) * y
    return out


def rel_l2(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("n,k,ne,e_lo,nl", [(1, 1, 4, 0, 4), (5, 2, 12, 4, 4), (40, 3, 16, 8, 8)])
def test_expert_call_matches_dense_float64(n, k, ne, e_lo, nl):
    x, ids, w, w13, w2 = setup(n, k, ne, e_lo, nl, seed=n)
    got = F.bf16_to_f32(OX.moe_ffn(x, ids, w, w13, w2, e_lo, act="bf16", block_m=4)).astype(np.float64)
    want = dense_reference(x, ids, w, w13, w2, e_lo)
    assert rel_l2(got, want) < 4e-3
    # per element: within a few bf16 ulps plus the h rounding the two orders may take differently
    assert np.all(np.abs(got - want) <= 2 ** -7 * np.abs(want) + 1e-3 * np.abs(want).max())


def test_gate_and_up_are_not_interchangeable():
    """The check above is sensitive to the [gate; up] order: swapping them moves the result."""
    x, ids, w, w13, w2 = setup(8, 2, 4, 0, 4, seed=3)
    swapped = np.concatenate([w13[:, I:], w13[:, :I]], axis=1)
    got = F.bf16_to_f32(OX.moe_ffn(x, ids, w, swapped, w2, 0, act="bf16")).astype(np.float64)
    assert rel_l2(got, dense_reference(x, ids, w, w13, w2, 0)) > 0.3


def test_no_local_pair_gives_exact_zeros():
    x, ids, w, w13, w2 = setup(16, 2, 8, 0, 4, seed=4)
    ids = ids % 4 + 4  # every pick on another rank
    assert not OX.moe_ffn(x, ids, w, w13, w2, 0).any()


def test_zero_weights_give_exact_zeros():
    x, ids, w, w13, w2 = setup(16, 2, 4, 0, 4, seed=5)
    out = OX.moe_ffn(x, ids, np.zeros_like(w), w13, w2, 0)
    assert np.all((out & 0x7FFF) == 0)  # +0 or -0


def test_repeated_tokens_give_identical_rows():
    x, ids, w, w13, w2 = setup(12, 2, 4, 0, 4, seed=6)
    x[5], ids[5], w[5] = x[2], ids[2], w[2]
    out = OX.moe_ffn(x, ids, w, w13, w2, 0)
    assert np.array_equal(out[5], out[2])


def test_power_of_two_weight_scaling_is_exact():
    x, ids, w, w13, w2 = setup(10, 1, 4, 0, 4, seed=7)
    a = F.bf16_to_f32(OX.moe_ffn(x, ids, w, w13, w2, 0))
    b = F.bf16_to_f32(OX.moe_ffn(x, ids, 4 * w, w13, w2, 0))
    assert np.array_equal(4 * a, b)


def test_mxfp8_activations_stay_close_to_bf16():
    x, ids, w, w13, w2 = setup(32, 2, 4, 0, 4, seed=8)
    a = F.bf16_to_f32(OX.moe_ffn(x, ids, w, w13, w2, 0, act="bf16"))
    for act in ("mxfp8", "fp8_1x128"):
        b = F.bf16_to_f32(OX.moe_ffn(x, ids, w, w13, w2, 0, act=act))
        assert 1e-4 < rel_l2(b, a) < 0.08, act  # quantized (not a no-op) but close


def test_finalize_matches_torch_fp32_ops():
    g = torch.Generator().manual_seed(9)
    n, k, rows = 24, 3, 80
    y = torch.randn(rows, H, generator=g).to(torch.bfloat16)
    w = torch.rand(n, k, generator=g)
    pos = torch.randint(-1, rows, (n * k,), generator=g, dtype=torch.int32)
    got = OX.finalize(bits(y), pos.numpy(), w.numpy(), n, k)
    acc = torch.zeros(n, H)
    for kk in range(k):
        p = pos.view(n, k)[:, kk]
        sel = p >= 0
        term = torch.zeros(n, H)
        term[sel] = w[sel, kk][:, None] * y[p[sel].long()].float()
        acc = torch.where(sel[:, None], acc + term, acc)
    assert np.array_equal(got, bits(acc.to(torch.bfloat16)))


@pytest.mark.parametrize("num_parts", [1, 2, 4])
def test_combine_matches_torch(num_parts):
    g = torch.Generator().manual_seed(10 + num_parts)
    parts = [torch.randn(7, H, generator=g).to(torch.bfloat16) for _ in range(num_parts)]
    shared = torch.randn(7, H, generator=g).to(torch.bfloat16)
    acc = parts[0].float()
    for p in parts[1:]:
        acc = acc + p.float()
    routed = parts[0].clone() if num_parts == 1 else acc.to(torch.bfloat16)
    assert np.array_equal(OX.combine([bits(p) for p in parts]), bits(routed))
    want = (routed.float() + shared.float()).to(torch.bfloat16)
    assert np.array_equal(OX.combine([bits(p) for p in parts], bits(shared)), bits(want))


# ---------------------------------------------------------------- SiTU
def _situ_math(g, u, a, l):
    """The SiTU formula evaluated independently, in float64 with the math module."""
    sig = 1.0 / (1.0 + math.exp(-g))
    return l * math.tanh(u / l) * a * math.tanh(g / a) * sig


def test_situ_matches_an_independent_evaluation():
    gen = torch.Generator().manual_seed(5)
    g = torch.randn(200, generator=gen) * 3
    u = torch.randn(200, generator=gen) * 3
    for a, l in ((2.0, 3.0), (0.5, 0.25), (7.0, 1.0)):
        got = OX.situ(g, u, a, l).double().numpy()
        want = np.array([_situ_math(float(gi), float(ui), a, l) for gi, ui in zip(g, u)])
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6 * a * l)


def test_situ_tends_to_swiglu_for_large_constants():
    """tanh(x / c) * c -> x as c grows, so SiTU -> u * g * sigmoid(g) = silu(g) * u."""
    gen = torch.Generator().manual_seed(6)
    g, u = torch.randn(500, generator=gen), torch.randn(500, generator=gen)
    big = OX.situ(g, u, 1e4, 1e4).double()
    swiglu = (g / (1 + torch.exp(-g)) * u).double()
    assert torch.allclose(big, swiglu, rtol=1e-5, atol=1e-7)


def test_situ_symmetries_and_bound():
    gen = torch.Generator().manual_seed(7)
    g, u = torch.randn(300, generator=gen) * 4, torch.randn(300, generator=gen) * 4
    a, l = 1.5, 0.75
    h = OX.situ(g, u, a, l)
    assert torch.equal(OX.situ(g, -u, a, l), -h)  # odd in the up value
    assert bool((h.abs() <= a * l).all())  # |tanh| <= 1 and sigmoid <= 1
    # the gate carries the sigmoid: swapping gate and up changes the value
    assert not torch.allclose(OX.situ(u, g, a, l), h, atol=1e-3)


def test_situ_layer_reduces_to_swiglu_layer():
    """The whole expert call with SiTU and huge constants equals the SwiGLU call."""
    x, ids, w, w13, w2 = setup(24, 2, 8, 0, 8, seed=9)
    a = OX.moe_ffn(x, ids, w, w13, w2, 0, act="bf16", activation="situ", act_alpha=1e5, act_limit=1e5)
    b = OX.moe_ffn(x, ids, w, w13, w2, 0, act="bf16")
    assert rel_l2(F.bf16_to_f32(a).astype(np.float64), F.bf16_to_f32(b).astype(np.float64)) < 1e-3


# ---------------------------------------------------------------- SwiGLU with a limit
def _swiglu_limit_math(g, u, l):
    """silu(min(g, l)) * clamp(u, -l, l), evaluated independently in float64."""
    gc = min(g, l)
    uc = max(-l, min(u, l))
    return gc / (1.0 + math.exp(-gc)) * uc


def test_swiglu_limit_matches_an_independent_evaluation():
    gen = torch.Generator().manual_seed(11)
    g = torch.randn(400, generator=gen) * 4
    u = torch.randn(400, generator=gen) * 4
    for l in (0.5, 2.0, 7.0):
        got = OX.swiglu_limit(g, u, l).double().numpy()
        want = np.array([_swiglu_limit_math(float(gi), float(ui), l) for gi, ui in zip(g, u)])
        assert np.allclose(got, want, rtol=1e-5, atol=1e-7)


def test_swiglu_limit_is_swiglu_where_no_clamp_binds():
    gen = torch.Generator().manual_seed(12)
    g, u = torch.randn(500, generator=gen), torch.randn(500, generator=gen)
    swiglu = OX.gate_up_act(g, u, "silu")
    assert torch.equal(OX.swiglu_limit(g, u, float("inf")), swiglu)
    l = 1.0
    inside = (g <= l) & (u.abs() <= l)
    assert bool(inside.any()) and bool((~inside).any())
    h = OX.swiglu_limit(g, u, l)
    assert torch.equal(h[inside], swiglu[inside])
    assert not torch.allclose(h[~inside], swiglu[~inside])


def test_swiglu_limit_saturation_symmetry_and_bound():
    gen = torch.Generator().manual_seed(13)
    g, u = torch.randn(300, generator=gen) * 5, torch.randn(300, generator=gen) * 5
    l = 1.5
    h = OX.swiglu_limit(g, u, l)
    # above the limit the gate saturates: any g > l gives the value at g = l
    big = g > l
    assert bool(big.any())
    assert torch.equal(h[big], OX.swiglu_limit(torch.full_like(g[big], l), u[big], l))
    # the gate is clamped above only: very negative gates still drive silu towards 0
    assert abs(float(OX.swiglu_limit(torch.tensor([-30.0]), torch.tensor([1.0]), l))) < 1e-9
    assert torch.equal(OX.swiglu_limit(g, -u, l), -h)  # odd in the up value
    silu_l = l / (1.0 + math.exp(-l))
    assert bool((h.abs() <= max(silu_l, 0.2785) * l + 1e-6).all())


def test_swiglu_limit_layer_reduces_to_swiglu_layer():
    """The whole expert call with a limit no value reaches equals the SwiGLU call bit for bit."""
    x, ids, w, w13, w2 = setup(24, 2, 8, 0, 8, seed=10)
    a = OX.moe_ffn(x, ids, w, w13, w2, 0, act="bf16", activation="swiglu_limit", act_limit=1e30)
    b = OX.moe_ffn(x, ids, w, w13, w2, 0, act="bf16")
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- shared expert
def _shared_float64(x, wg, wu, wd):
    """The dense SwiGLU shared expert in float64 numpy, element formulas written out:
    h_j = g_j / (1 + exp(-g_j)) * u_j with g = Wg x, u = Wu x; out = Wd h."""
    xf = x.double().numpy()
    g = np.einsum("ih,th->ti", wg.double().numpy(), xf)
    u = np.einsum("ih,th->ti", wu.double().numpy(), xf)
    h = g / (1.0 + np.exp(-g)) * u
    return np.einsum("hi,ti->th", wd.double().numpy(), h)


def _shared_case(n=24, hidden=H, inter=96, seed=3):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, hidden, generator=g).to(torch.bfloat16)
    wg = (torch.randn(inter, hidden, generator=g) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(inter, hidden, generator=g) * 0.05).to(torch.bfloat16)
    wd = (torch.randn(hidden, inter, generator=g) * 0.05).to(torch.bfloat16)
    return x, wg, wu, wd


def test_shared_mlp_matches_float64_dense_swiglu():
    """bf16(fp32 evaluation) against bf16(float64 evaluation): equal bits except where the
    float64 value sits within fp32 noise of a bf16 rounding boundary, never more than one
    bf16 step apart. inter != hidden, so a transposed operand cannot pass."""
    x, wg, wu, wd = _shared_case()
    got = bits(OX.shared_mlp(x, wg, wu, wd)).astype(np.int32)
    want = bits(torch.from_numpy(_shared_float64(x, wg, wu, wd)).float().to(torch.bfloat16)).astype(np.int32)
    assert np.mean(got == want) > 0.99
    assert np.abs(got - want).max() <= 1


def test_shared_mlp_sensitivity_and_zeros():
    x, wg, wu, wd = _shared_case(seed=4)
    ref = bits(OX.shared_mlp(x, wg, wu, wd))
    assert np.mean(bits(OX.shared_mlp(x, wu, wg, wd)) == ref) < 0.1  # gate and up swapped
    assert not bits(OX.shared_mlp(x, wg, torch.zeros_like(wu), wd)).any()  # up = 0 -> exact zeros
    assert not bits(OX.shared_mlp(torch.zeros_like(x), wg, wu, wd)).any()  # silu(0) * 0 = 0
    # one token, one hidden unit: out = wd[:, 0] * silu(g) * u in closed form
    x1 = x[:1]
    wg1, wu1, wd1 = wg[:1], wu[:1], wd[:, :1]
    g1 = float((wg1.double() @ x1.double().T).item())
    u1 = float((wu1.double() @ x1.double().T).item())
    want = wd1.double()[:, 0] * (g1 / (1 + math.exp(-g1)) * u1)
    got = OX.shared_mlp(x1, wg1, wu1, wd1)[0].double()
    assert torch.allclose(got, want, rtol=8e-3, atol=1e-6)
