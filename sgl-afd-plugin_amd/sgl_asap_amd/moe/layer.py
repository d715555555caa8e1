"""The MoE layer of an attention rank whose routed experts run on the FFN ranks.

Same constructor and ``forward`` as ``AsapMoE`` in
``python/sgl_asap_plugin/srt/layers/moe/ep_moe/layer.py:24-94``: a FusedMoE without expert
weights, whose ``forward(hidden_states, topk_output, pre_quant_input=None)`` hands the
routed experts to the F ranks through ``AsapDispatcher``. Fused shared experts are refused
(:54-58); routed scaling is expected in the top-k weights
(``should_fuse_routed_scaling_factor_in_topk``).

The shared experts stay on the attention rank. When a ``shared_experts`` callable is given,
it runs on the compute stream between dispatch and combine (the ordering the reference's
single-batch overlap installs, ``srt/batch_overlap/single_batch_overlap.py:109-134``) and
its output is added inside the combine kernel.
"""

from __future__ import annotations

from typing import Callable, Optional

import torch

from .dispatcher import AsapDispatcher


class AsapMoE(torch.nn.Module):
    should_fuse_routed_scaling_factor_in_topk = True
    quant_method = None

    def __init__(
        self,
        num_experts: int,
        hidden_size: int,
        intermediate_size: int,
        layer_id: int,
        top_k: Optional[int] = None,
        num_fused_shared_experts: int = 0,
        params_dtype: Optional[torch.dtype] = None,
        routed_scaling_factor: Optional[float] = None,
        shared_experts: Optional[Callable[[torch.Tensor], torch.Tensor]] = None,
        **kwargs,
    ):
        super().__init__()
        if num_fused_shared_experts:
            raise ValueError("ASAP keeps the shared experts on the attention ranks: disable shared experts fusion")
        self.num_experts = num_experts
        self.num_local_experts = 0
        self.num_fused_shared_experts = 0
        self.top_k = top_k
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.layer_id = layer_id
        self.params_dtype = params_dtype
        self.routed_scaling_factor = routed_scaling_factor
        self.dispatcher = AsapDispatcher(layer_id)
        self.shared_experts = shared_experts

    def forward(self, hidden_states: torch.Tensor, topk_output, pre_quant_input=None, micro_batch: Optional[int] = None):
        # The FFN ranks run the routed experts between dispatch and combine; the shared
        # experts run here meanwhile.
        dispatch_output = self.dispatcher.dispatch(hidden_states, topk_output, micro_batch)
        shared = self.shared_experts(hidden_states) if self.shared_experts is not None else None
        return self.dispatcher.combine(dispatch_output, shared)
