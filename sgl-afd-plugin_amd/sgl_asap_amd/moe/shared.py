"""The attention rank's shared expert: a dense bf16 SwiGLU MLP.

In the reference the shared experts stay on the attention rank and are the model's own MLP
(SGLang's, not part of the plugin); their output is added to the routed partial sums after
the combine (``python/sgl_asap_plugin/srt/batch_overlap/operations_strategy.py:106-111``,
ordering in ``srt/batch_overlap/single_batch_overlap.py:109-134``). This module is that MLP
for the one-GPU loop and its benchmark: plain library GEMMs (hipBLASLt through torch) in
bf16, with the gate and up projections in one matrix.

    out = W_down . (silu(W_gate . x) * (W_up . x))

The add itself is fused into the combine kernel (``afd_combine``'s ``shared`` argument).
"""

from __future__ import annotations

import torch


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
        gate, up = torch.mm(x, self.w_gate_up.t()).split(self.intermediate_size, dim=1)
        return torch.mm(torch.nn.functional.silu(gate) * up, self.w_down.t())
