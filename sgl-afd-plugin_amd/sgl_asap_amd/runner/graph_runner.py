"""HIP graphs of the expert calls of an FFN rank, per (layer, token bucket, output buffer).

Same rules as ``python/sgl_asap_plugin/srt/model_executor/runner/ffn_cuda_graph_runner.py``:
buckets are the powers of two below ``max_tokens`` plus ``max_tokens`` (:36-39); padding rows
route to ``pad_id`` = an expert of another rank when the rank is partial, else the first
local expert with weight 0 (:40-42, :88-90); two static output buffers, one graph per
(layer, bucket, buffer) (:48-66); ``run`` copies the job's rows into the static inputs, pads
them to the bucket, replays, and returns a view of the output buffer, or None when the job
is larger than the largest bucket (:75-92).

With fp8 activations on the wire (``act`` "mxfp8" / "fp8_1x128") the static inputs are the
e4m3 codes and their scales and the graphs capture ``forward_q``.

A graph replay removes the per-job host cost of the eager call (argument checks, the
ctypes call and its kernel launches). Our kernels read the device-side row-tile count the
router writes, so a bucket's graph serves any job size up to the bucket. The stream memops
of the transport stay outside the graphs: their values are fixed at capture time.
"""

from __future__ import annotations

import bisect
import time
from typing import Dict, Optional

import torch

from ..moe.experts import act_scale_shape
from ..moe.topk import StandardTopKOutput


def graph_buckets(max_tokens: int) -> list:
    b = [1 << i for i in range(max_tokens.bit_length()) if 1 << i < max_tokens]
    return b + [max_tokens]


def pad_id_for(local: range, num_experts: int) -> int:
    return local.stop % num_experts if len(local) < num_experts else local.start


class FfnGraphRunner:
    def __init__(self, experts: Dict[int, torch.nn.Module], max_tokens: int, local: range, act: str = "bf16"):
        first = next(iter(experts.values()))
        hidden, topk, num_experts = first.hidden_size, first.top_k, first.num_experts
        self.buckets = graph_buckets(max_tokens)
        self.pad_id = pad_id_for(local, num_experts)
        device = torch.cuda.current_device()
        n = self.buckets[-1]
        if act == "bf16":
            self.x = (torch.zeros(n, hidden, dtype=torch.bfloat16, device=device),)
        else:
            shape, dtype = act_scale_shape(act, n, hidden)
            # zero codes with scale 1.0 (UE8M0 127): padding rows stay finite
            self.x = (torch.zeros(n, hidden, dtype=torch.uint8, device=device),
                      torch.full(shape, 127 if act == "mxfp8" else 1.0, dtype=dtype, device=device))
        self.ids = torch.full((n, topk), self.pad_id, dtype=torch.int32, device=device)
        self.w = torch.zeros(n, topk, dtype=torch.float32, device=device)
        self.outs = [torch.zeros(n, hidden, dtype=torch.bfloat16, device=device) for _ in range(2)]
        self.graphs: Dict[tuple, torch.cuda.CUDAGraph] = {}
        tic = time.perf_counter()
        pool = torch.cuda.graph_pool_handle()
        stream = torch.cuda.Stream()
        for b in reversed(self.buckets):
            topk_output = StandardTopKOutput(self.w[:b], self.ids[:b], None)
            x = tuple(t[:b] for t in self.x)
            for layer_id, layer in experts.items():
                call = layer if act == "bf16" else layer.forward_q
                stream.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(stream):  # first call outside the capture
                    call(*x, topk_output, out=self.outs[0][:b])
                torch.cuda.current_stream().wait_stream(stream)
                for k, out in enumerate(self.outs):
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, pool=pool, stream=stream):
                        call(*x, topk_output, out=out[:b])
                    self.graphs[(layer_id, b, k)] = graph
        torch.cuda.synchronize()
        self.capture_s = time.perf_counter() - tic

    def run(self, layer_id: int, x, topk_ids, topk_weights, buffer: int = 0) -> Optional[torch.Tensor]:
        """The expert output of the job's rows in output buffer ``buffer`` (0 or 1), or None
        if the job is larger than the largest bucket (the caller runs it eagerly). ``x`` is a
        bf16 tensor, or a tuple of the rows' tensors in the runner's activation format."""
        x = x if isinstance(x, tuple) else (x,)
        if len(x) != len(self.x):
            raise ValueError(f"the graphs take {len(self.x)} activation tensors, got {len(x)}")
        n = topk_ids.shape[0]
        i = bisect.bisect_left(self.buckets, n)
        if i == len(self.buckets):
            return None
        b = self.buckets[i]
        for dst, src in zip(self.x, x):
            dst[:n].copy_(src)
        self.ids[:n].copy_(topk_ids)
        self.w[:n].copy_(topk_weights)
        if n < b:
            self.ids[n:b].fill_(self.pad_id)
            self.w[n:b].zero_()
        self.graphs[(layer_id, b, buffer)].replay()
        return self.outs[buffer][:n]
