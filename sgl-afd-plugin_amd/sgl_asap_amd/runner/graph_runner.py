"""HIP graphs of the expert calls of an FFN rank, one per (layer, token bucket).

Replaces ``python/sgl_asap_plugin/srt/model_executor/runner/ffn_cuda_graph_runner.py``. The
buckets are the reference's: the powers of two below ``max_tokens`` plus ``max_tokens``
(:36-39), and a job larger than the largest bucket runs eagerly (``run`` returns None,
:75-92). The reference copies a job's rows into static input buffers, pads them to the
bucket with a pad expert (:40-42, :88-90), replays into one of two static output buffers
(:48-66) and copies the result out. Here each graph captures ``afd_moe_ffn_job``, whose
launches read the job from a device descriptor when they run: ``run`` writes the job's
pointers and size into the descriptor (one small launch) and replays. The kernels then read
the rows in place (the RecvArena), do no work for the tokens the job lacks, and write the
output where the caller says (A's result segment), so nothing is copied in or out; the bucket
only bounds the grids. Jobs of several rows (a TP group) are concatenated first, and without
an ``out`` their output lands in one of two internal buffers used in turn, as in the
reference.

With fp8 activations on the wire (``act`` "mxfp8" / "fp8_1x128") the descriptor carries the
e4m3 codes and their scales instead of bf16 rows.

The stream memops of the transport stay outside the graphs: their values are fixed at
capture time.
"""

from __future__ import annotations

import bisect
import ctypes
import time
from typing import Dict, Optional

import torch

from .. import _lib
from ..moe.experts import new_job_desc, set_job


def graph_buckets(max_tokens: int) -> list:
    b = [1 << i for i in range(max_tokens.bit_length()) if 1 << i < max_tokens]
    return b + [max_tokens]


class FfnGraphRunner:
    def __init__(self, experts: Dict[int, torch.nn.Module], max_tokens: int, local: range, act: str = "bf16"):
        first = next(iter(experts.values()))
        hidden = first.hidden_size
        self.buckets = graph_buckets(max_tokens)
        self.local = local
        self.quantized = act != "bf16"
        device = torch.cuda.current_device()
        self.desc = new_job_desc(device)  # n = 0 until the first job: a replay then does nothing
        # the runner's own workspace (its graphs capture its pointer), large enough for every layer
        self.ws = torch.empty(max(layer.layout["total"] for layer in experts.values()), dtype=torch.uint8,
                              device=device)
        self.outs = [torch.zeros(max_tokens, hidden, dtype=torch.bfloat16, device=device) for _ in range(2)]
        self.graphs: Dict[tuple, torch.cuda.CUDAGraph] = {}
        tic = time.perf_counter()
        pool = torch.cuda.graph_pool_handle()
        stream = torch.cuda.Stream()
        for b in reversed(self.buckets):
            for layer_id, layer in experts.items():
                stream.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(stream):  # first call outside the capture
                    layer.call_job(self.desc, b, self.quantized, ws=self.ws)
                torch.cuda.current_stream().wait_stream(stream)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=pool, stream=stream):
                    layer.call_job(self.desc, b, self.quantized, ws=self.ws)
                self.graphs[(layer_id, b)] = graph
        torch.cuda.synchronize()
        self.capture_s = time.perf_counter() - tic
        self._job = _lib.AfdJob()  # host staging of run_ptrs' descriptor writes

    def run_ptrs(self, layer_id: int, n: int, x_ptr: int, xs_ptr: int, ids_ptr: int, w_ptr: int,
                 out_ptr: int) -> bool:
        """``run`` on raw device pointers (the serving loop's arena records): writes the job into
        the descriptor and replays the bucket's graph on the current stream; False, doing
        nothing, if n is above the largest bucket. bf16 rows at x_ptr (xs_ptr = 0), or, for a
        runner of quantized rows, the e4m3 codes at x_ptr and their scales at xs_ptr."""
        i = bisect.bisect_left(self.buckets, n)
        if i == len(self.buckets) or n < 1:
            return False
        if bool(xs_ptr) != self.quantized:
            raise ValueError(f"the graphs take {'quantized' if self.quantized else 'bf16'} rows")
        j = self._job
        if self.quantized:
            j.x, j.xq, j.xs = None, x_ptr, xs_ptr
        else:
            j.x, j.xq, j.xs = x_ptr, None, None
        j.ids, j.w, j.out, j.n = ids_ptr, w_ptr, out_ptr, n
        _lib.call("afd_job_set", self.desc.data_ptr(), ctypes.byref(j), torch.cuda.current_stream().cuda_stream)
        self.graphs[(layer_id, self.buckets[i])].replay()
        return True

    def run(self, layer_id: int, x, topk_ids, topk_weights, buffer: int = 0,
            out: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
        """Enqueue the expert call of the job's rows on the current stream and return its
        output: ``out`` if given (bf16 [n, H]), else output buffer ``buffer`` (0 or 1). None if
        the job is larger than the largest bucket (the caller runs it eagerly). ``x`` is a bf16
        tensor, or the tuple of the rows' tensors in the runner's activation format. The
        inputs must stay alive until the replay has run (stream order)."""
        x = x if isinstance(x, tuple) else (x,)
        if len(x) != (2 if self.quantized else 1):
            raise ValueError(f"the graphs take {2 if self.quantized else 1} activation tensors, got {len(x)}")
        n = topk_ids.shape[0]
        i = bisect.bisect_left(self.buckets, n)
        if i == len(self.buckets):
            return None
        if out is None:
            out = self.outs[buffer][:n]
        ids = topk_ids.to(torch.int32).contiguous()
        w = topk_weights.to(torch.float32).contiguous()
        if self.quantized:
            set_job(self.desc, xq=x[0].contiguous(), xs=x[1].contiguous(), ids=ids, w=w, out=out)
        else:
            set_job(self.desc, x=x[0].contiguous(), ids=ids, w=w, out=out)
        self.graphs[(layer_id, self.buckets[i])].replay()
        return out
