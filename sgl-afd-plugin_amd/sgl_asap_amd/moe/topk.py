"""The top-k output the expert call takes, with the reference's field names.

The reference passes SGLang's ``StandardTopKOutput(topk_weights, topk_ids, router_logits)``
(``python/sgl_asap_plugin/srt/managers/scheduler.py:410-412``;
``srt/model_executor/runner/ffn_cuda_graph_runner.py:57``). SGLang is not a dependency here,
so the same three-field tuple is defined locally; any object with ``topk_weights`` and
``topk_ids`` attributes is accepted where it is consumed.
"""

from __future__ import annotations

from typing import NamedTuple, Optional

import torch


class StandardTopKOutput(NamedTuple):
    topk_weights: torch.Tensor  # f32 [n, k], routed scaling already applied
    topk_ids: torch.Tensor  # i32 [n, k], global expert ids
    router_logits: Optional[torch.Tensor] = None


def format_is_standard(topk_output) -> bool:
    """``TopKOutputChecker.format_is_standard`` as the dispatcher uses it
    (``srt/layers/moe/token_dispatcher/asap.py:60``): explicit ids and weights."""
    return hasattr(topk_output, "topk_ids") and hasattr(topk_output, "topk_weights")
