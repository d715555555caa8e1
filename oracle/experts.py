"""fp32 CPU restatement of the F-side expert call, the finalize and the A-side combine
(test infrastructure; also the timed ``cpu_baseline`` of bench.py).

What it restates:
* the expert call ``FusedMoE(x, StandardTopKOutput(w, ids, None))``
  (``python/sgl_asap_plugin/srt/managers/scheduler.py:410-412``):
  ``out[t] = sum_{kk: ids[t,kk] local} w[t,kk] * W2_e . silu(Wg_e . x_t) * (Wu_e . x_t)``
  with W13 = [gate(I); up(I)] (``srt/models/deepseek_v4.py:132-137``), top-k weights that
  already carry the routed scaling (``srt/layers/moe/ep_moe/layer.py:29-36``), rows with no
  local expert = 0, output bf16;
* the activation quantization the MXFP4 method applies before gemm1
  (``srt/layers/quantization/mxfp4_flashinfer_trtllm_moe.py:49-61``: MXFP8 by default);
* the A-side combine ``AsapBuffer.recv`` (``srt/layers/moe/token_dispatcher/asap.py:174-184``)
  and the plain shared-expert add (``srt/layers/moe/ep_moe/layer.py:29-33``,
  ``srt/batch_overlap/operations_strategy.py:106-111``).

Rounding points (the GPU path applies the same quantizers at the same places, so only
fp32 summation order differs):
  x -> MXFP8 (or FP8 1x128) ; gemm1 fp32 ; h = silu(g) * u fp32 ; h -> MXFP8 (or FP8
  1x128) ; gemm2 fp32 ; y -> bf16 ; out = bf16(sum over kk in order of fp32(w) * fp32(y)),
  each product and each sum rounded to fp32 separately (no fused multiply-add).

Pinned by: the closed-form special cases (all ids non-local -> exact zeros; w = 0 -> zeros;
one token + one expert -> a plain dense MLP computed independently in float64; identical
tokens -> identical rows) and by the bit-exact combine formula; see tests/test_oracle_experts.py.
"""

from __future__ import annotations

import numpy as np
import torch

from . import formats as F
from .routing import route


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _silu(g: torch.Tensor) -> torch.Tensor:
    return g / (1.0 + torch.exp(-g))


def situ(g: torch.Tensor, u: torch.Tensor, alpha: float, limit: float) -> torch.Tensor:
    """SiTU of the gate and up values: ``limit * tanh(u / limit) * alpha * tanh(g / alpha) *
    sigmoid(g)``, the function the reference's SiTU hook runs: the FlashInfer kernel computes
    ``beta * tanh(x0 / beta) * alpha * tanh(x1 / alpha) * sigmoid(x1)`` with x0 the up and x1
    the gate row, alpha = gemm1_alpha (SiTU's beta) and beta = gemm1_beta (its linear_beta)
    (python/sgl_asap_plugin/srt/layers/quantization/mxfp4_flashinfer_trtllm_moe.py:13-16,
    call at :67-98). fp32 torch.

    Pinned (tests/test_oracle_experts.py): values against an independent math-module
    evaluation, the limit alpha, limit -> inf (SwiGLU: silu(g) * u), odd symmetry in u,
    |h| <= alpha * limit, and that g alone carries the sigmoid."""
    return (limit * torch.tanh(u / limit)) * (alpha * torch.tanh(g / alpha)) * torch.sigmoid(g)


def swiglu_limit(g: torch.Tensor, u: torch.Tensor, limit: float) -> torch.Tensor:
    """SwiGLU with a limit: ``silu(min(g, limit)) * clamp(u, -limit, limit)``, DeepSeek-V4's
    ``swiglu_limit``, which the reference passes to FusedMoE
    (python/sgl_asap_plugin/srt/models/deepseek_v4.py:63) and SGLang hands to the MoE kernel
    as gemm1_clamp_limit; the clamped-SwiGLU form of the public DeepSeek-V4 and TRT-LLM
    expert code (gate clamped above only, up on both sides). fp32 torch.

    Pinned (tests/test_oracle_experts.py): equal to SwiGLU wherever no clamp binds and for an
    infinite limit, values against an independent math-module evaluation of the clamped form,
    saturation in g above the limit, odd symmetry in u and the bound
    |h| <= max(silu(limit), 0.2785) * limit."""
    return _silu(torch.clamp(g, max=limit)) * torch.clamp(u, -limit, limit)


def gate_up_act(g: torch.Tensor, u: torch.Tensor, activation: str = "silu", alpha=None, limit=None):
    """h of the gate_up output: SwiGLU silu(g) * u (SGLang's default activation), SwiGLU with
    a limit ("swiglu_limit") or SiTU."""
    if activation == "silu":
        return _silu(g) * u
    if activation == "swiglu_limit":
        return swiglu_limit(g, u, limit)
    if activation == "situ":
        return situ(g, u, alpha, limit)
    raise NotImplementedError(activation)


def quantize_act(x_f32: np.ndarray, act: str) -> np.ndarray:
    """Apply the activation quantizer and return the dequantized fp32 values."""
    if act == "mxfp8":
        q, s = F.mx_quantize(x_f32, "e4m3")
        return F.mx_dequantize(q, s, "e4m3")
    if act == "fp8_1x128":
        q, s = F.fp8_group_quantize(x_f32)
        return F.fp8_group_dequantize(q, s)
    if act == "bf16":
        return F.bf16_to_f32(F.f32_to_bf16(x_f32))
    raise ValueError(act)


def finalize(y_bf16: np.ndarray, pair_pos: np.ndarray, w: np.ndarray, n: int, k: int) -> np.ndarray:
    """out[t] = bf16(sum_kk fp32(w[t,kk]) * fp32(y[pair_pos[t*k+kk]])), products and sums
    rounded to fp32 one at a time, kk ascending; non-local pairs skipped. -> uint16 bf16 bits."""
    y = F.bf16_to_f32(y_bf16)
    hdim = y.shape[1]
    acc = np.zeros((n, hdim), dtype=np.float32)
    pos = pair_pos.reshape(n, k)
    w = np.asarray(w, dtype=np.float32).reshape(n, k)
    for kk in range(k):
        sel = pos[:, kk] >= 0
        prod = (w[sel, kk][:, None] * y[pos[sel, kk]]).astype(np.float32)
        acc[sel] = (acc[sel] + prod).astype(np.float32)
    return F.f32_to_bf16(acc)


def expert_rows(x_deq: np.ndarray, sorted_pairs: np.ndarray, k: int) -> np.ndarray:
    """Gather dequantized activation rows in padded expert order (pad rows = 0)."""
    rows = np.zeros((sorted_pairs.shape[0], x_deq.shape[1]), dtype=np.float32)
    valid = sorted_pairs >= 0
    rows[valid] = x_deq[sorted_pairs[valid] // k]
    return rows


def moe_ffn(
    x_bf16: torch.Tensor,
    ids: np.ndarray,
    w: np.ndarray,
    w13_deq: np.ndarray,
    w2_deq: np.ndarray,
    e_lo: int,
    act: str = "mxfp8",
    block_m: int = 128,
    return_parts: bool = False,
    activation: str = "silu",
    act_alpha=None,
    act_limit=None,
):
    """One job through one F rank's experts.

    x_bf16: torch bf16 [n, H] (CPU). ids int32 [n, k] global ids. w fp32 [n, k].
    w13_deq: fp32 [E, 2I, H] logical rows [gate; up], dequantized. w2_deq: fp32 [E, H, I].
    act: activation quantizer applied to x and to h ("mxfp8", "fp8_1x128" or "bf16").
    activation: the gate_up activation, "silu" (SwiGLU), "swiglu_limit" with act_limit, or
    "situ" with act_alpha, act_limit.
    Returns bf16 bits uint16 [n, H] (and the intermediates when return_parts).
    """
    n, hdim = x_bf16.shape
    k = ids.shape[1]
    num_local, two_i, _ = w13_deq.shape
    inter = two_i // 2
    r = route(ids, e_lo, num_local, block_m)
    x_f32 = F.bf16_to_f32(_bf16_bits(x_bf16))
    x_deq = quantize_act(x_f32, act)
    a_rows = expert_rows(x_deq, r["sorted_pairs"], k)
    np_pad = a_rows.shape[0]
    y = np.zeros((np_pad, hdim), dtype=np.float32)
    h_all = np.zeros((np_pad, inter), dtype=np.float32)
    poff = r["padded_offsets"]
    for e in range(num_local):
        lo, cnt = int(poff[e]), int(r["counts"][e])
        if cnt == 0:
            continue
        a = torch.from_numpy(a_rows[lo : lo + cnt])
        w13 = torch.from_numpy(w13_deq[e])
        gu = a @ w13.T
        g, u = gu[:, :inter], gu[:, inter:]
        h = gate_up_act(g, u, activation, act_alpha, act_limit).numpy()
        h_deq = quantize_act(h, act)
        h_all[lo : lo + cnt] = h_deq
        y[lo : lo + cnt] = (torch.from_numpy(h_deq) @ torch.from_numpy(w2_deq[e]).T).numpy()
    y_bf16 = F.f32_to_bf16(y)
    out = finalize(y_bf16, r["pair_pos"], w, n, k)
    if return_parts:
        return out, {"route": r, "y_bf16": y_bf16, "h": h_all, "x_deq": x_deq}
    return out


def combine(parts: list, shared=None) -> np.ndarray:
    """A-side combine: bf16(sum_f fp32(part_f)) in f order (one part: a copy), then
    bf16(fp32(routed) + fp32(shared)) when a shared-expert output is given.
    parts / shared: uint16 bf16 bits of equal shape. -> uint16 bits."""
    if len(parts) == 1:
        routed = np.array(parts[0], dtype=np.uint16, copy=True)
    else:
        acc = F.bf16_to_f32(parts[0]).astype(np.float32)
        for p in parts[1:]:
            acc = (acc + F.bf16_to_f32(p)).astype(np.float32)
        routed = F.f32_to_bf16(acc)
    if shared is None:
        return routed
    return F.f32_to_bf16((F.bf16_to_f32(routed) + F.bf16_to_f32(shared)).astype(np.float32))


def shared_mlp(x_bf16: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor) -> torch.Tensor:
    """Dense SwiGLU shared expert in fp32 on the CPU: bf16(wd . (silu(wg . x) * (wu . x)))."""
    x = x_bf16.float()
    h = _silu(x @ wg.float().T) * (x @ wu.float().T)
    return (h @ wd.float().T).to(torch.bfloat16)
