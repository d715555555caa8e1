"""HIP graphs of the expert calls of an FFN rank, per (layer, token bucket, output buffer).

Same rules as ``python/sgl_asap_plugin/srt/model_executor/runner/ffn_cuda_graph_runner.py``:
buckets are the powers of two below ``max_tokens`` plus ``max_tokens`` (:36-39); padding rows
route to ``pad_id`` = an expert of another rank when the rank is partial, else the first
local expert with weight 0 (:40-42, :88-90); two static output buffers, one graph per
(layer, bucket, buffer) (:48-66); ``run`` copies the job's rows into the static inputs, pads
them to the bucket, replays, and returns a view of the output buffer, or None when the job
is larger than the largest bucket (:75-92).

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

from ..moe.topk import StandardTopKOutput


def graph_buckets(max_tokens: int) -> list:
    b = [1 << i for i in range(max_tokens.bit_length()) if 1 << i < max_tokens]
    return b + [max_tokens]


def pad_id_for(local: range, num_experts: int) -> int:
    return local.stop % num_experts if len(local) < num_experts else local.start


class FfnGraphRunner:
    def __init__(self, experts: Dict[int, torch.nn.Module], max_tokens: int, local: range):
        first = next(iter(experts.values()))
        hidden, topk, num_experts = first.hidden_size, first.top_k, first.num_experts
        self.buckets = graph_buckets(max_tokens)
        self.pad_id = pad_id_for(local, num_experts)
        device = torch.cuda.current_device()
        n = self.buckets[-1]
        self.x = torch.zeros(n, hidden, dtype=torch.bfloat16, device=device)
        self.ids = torch.full((n, topk), self.pad_id, dtype=torch.int32, device=device)
        self.w = torch.zeros(n, topk, dtype=torch.float32, device=device)
        self.outs = [torch.zeros(n, hidden, dtype=torch.bfloat16, device=device) for _ in range(2)]
        self.graphs: Dict[tuple, torch.cuda.CUDAGraph] = {}
        tic = time.perf_counter()
        pool = torch.cuda.graph_pool_handle()
        stream = torch.cuda.Stream()
        for b in reversed(self.buckets):
            topk_output = StandardTopKOutput(self.w[:b], self.ids[:b], None)
            for layer_id, layer in experts.items():
                stream.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(stream):  # first call outside the capture
                    layer(self.x[:b], topk_output, out=self.outs[0][:b])
                torch.cuda.current_stream().wait_stream(stream)
                for k, out in enumerate(self.outs):
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, pool=pool, stream=stream):
                        layer(self.x[:b], topk_output, out=out[:b])
                    self.graphs[(layer_id, b, k)] = graph
        torch.cuda.synchronize()
        self.capture_s = time.perf_counter() - tic

    def run(self, layer_id: int, x, topk_ids, topk_weights, buffer: int = 0) -> Optional[torch.Tensor]:
        """The expert output of the job's rows in output buffer ``buffer`` (0 or 1), or None
        if the job is larger than the largest bucket (the caller runs it eagerly)."""
        n = x.shape[0]
        i = bisect.bisect_left(self.buckets, n)
        if i == len(self.buckets):
            return None
        b = self.buckets[i]
        self.x[:n].copy_(x)
        self.ids[:n].copy_(topk_ids)
        self.w[:n].copy_(topk_weights)
        if n < b:
            self.ids[n:b].fill_(self.pad_id)
            self.w[n:b].zero_()
        self.graphs[(layer_id, b, buffer)].replay()
        return self.outs[buffer][:n]
