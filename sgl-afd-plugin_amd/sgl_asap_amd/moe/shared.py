"""The attention rank's shared expert: a dense bf16 SwiGLU MLP.

In the reference the shared experts stay on the attention rank and are the model's own MLP
(SGLang's, not part of the plugin); their output is added to the routed partial sums after
the combine (``python/sgl_asap_plugin/srt/batch_overlap/operations_strategy.py:106-111``,
ordering in ``srt/batch_overlap/single_batch_overlap.py:109-134``). This module is that MLP
for the one-GPU loop and its benchmark: plain library GEMMs (hipBLASLt through torch) in
bf16, with the gate and up projections in one matrix, and between them the activation as one
HBM-bound kernel (``afd_silu_mul``, SGLang's fused SiluAndMul; silu and the product as two
torch kernels on the strided gate half took 164 us of a loop layer).

    out = W_down . bf16(silu(W_gate . x) * (W_up . x))

The add itself is fused into the combine kernel (``afd_combine``'s ``shared`` argument).
"""

from __future__ import annotations

import torch

from .. import _lib


class SharedExpertMLP(torch.nn.Module):
    """``w_gate_up`` bf16 [2I, H] = [gate; up] rows, ``w_down`` bf16 [H, I]."""

    def __init__(self, w_gate_up: torch.Tensor, w_down: torch.Tensor):
        super().__init__()
        two_i, hidden = w_gate_up.shape
        if two_i % 2 or tuple(w_down.shape) != (hidden, two_i // 2):
            raise ValueError(f"w_gate_up {tuple(w_gate_up.shape)} and w_down {tuple(w_down.shape)} "
                             "do not form one SwiGLU MLP")
        if w_gate_up.dtype != torch.bfloat16 or w_down.dtype != torch.bfloat16:
            raise TypeError("the shared expert runs in bf16")
        self.hidden_size, self.intermediate_size = hidden, two_i // 2
        self.w_gate_up = w_gate_up.contiguous()
        self.w_down = w_down.contiguous()

    @classmethod
    def random(cls, hidden: int, inter: int, generator: torch.Generator, device, std: float = 0.02):
        """Weights ~ N(0, std) drawn in fp32 on ``device`` (gate_up first), rounded to bf16."""
        w_gu = torch.randn(2 * inter, hidden, generator=generator, device=device) * std
        w_d = torch.randn(hidden, inter, generator=generator, device=device) * std
        return cls(w_gu.to(torch.bfloat16), w_d.to(torch.bfloat16))

    @property
    def w_gate(self) -> torch.Tensor:
        return self.w_gate_up[: self.intermediate_size]

    @property
    def w_up(self) -> torch.Tensor:
        return self.w_gate_up[self.intermediate_size :]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != self.hidden_size:
            raise TypeError(f"expected bf16 [n, {self.hidden_size}], got {x.dtype} {tuple(x.shape)}")
        gate_up = torch.mm(x, self.w_gate_up.t())
        return torch.mm(silu_mul(gate_up), self.w_down.t())


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """bf16(silu(gate) * up) of bf16 [n, 2I] rows [gate | up] on their device's current stream:
    SGLang's SiluAndMul, as ``afd_silu_mul``."""
    if gate_up.dtype != torch.bfloat16 or gate_up.dim() != 2 or gate_up.shape[1] % 2:
        raise TypeError(f"expected bf16 [n, 2I], got {gate_up.dtype} {tuple(gate_up.shape)}")
    gate_up = gate_up.contiguous()
    n, inter = gate_up.shape[0], gate_up.shape[1] // 2
    out = torch.empty(n, inter, dtype=torch.bfloat16, device=gate_up.device)
    _lib.call("afd_silu_mul", gate_up.data_ptr(), n, inter, out.data_ptr(),
              torch.cuda.current_stream(gate_up.device).cuda_stream)
    return out
