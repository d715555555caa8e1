"""The F rank's job handler: routed experts per MoE layer, served job by job.

Follows ``FfnScheduler`` in ``python/sgl_asap_plugin/srt/managers/scheduler.py``:
``local_experts`` (:206-218), ``warmup`` over every power of two up to n_max with the seeded
generator (:329-351), ``run_job`` (:387-436: row views of the RecvArena, the graph runner or
the eager expert call, a reply stream that waits for the experts, ``reply`` per row, the two
graph output buffers reused in turn behind ``reply_free`` events), ``rows_of`` (:438-450) and
``JobTimer`` (:109-159: host launch time and GPU expert / reply times per power-of-two
bucket, from events read lazily).

Differences on one GPU: the experts run on the scheduler's own stream, which first parks
on the job's doorbells (``FfnServer.wait_rows``), so the host never waits; an eager job
writes its output straight into A's result segment, so its reply is the done flag alone.
With fp8 activations on the wire (``Geometry.act``) the rows arrive as e4m3 codes plus
scales and the job runs the expert call on them as they are (``forward_q``).
"""

from __future__ import annotations

import collections
import statistics
import time
from typing import Dict, Optional

import torch

from ..moe.experts import act_scale_shape
from ..moe.topk import StandardTopKOutput
from .graph_runner import FfnGraphRunner, graph_buckets


def local_experts(ep_rank: int, ep_size: int, num_experts: int) -> range:
    """The routed experts of this EP rank: num_experts // ep_size contiguous global ids."""
    per_rank = num_experts // ep_size
    return range(ep_rank * per_rank, (ep_rank + 1) * per_rank)


class JobTimer:
    """Per power-of-two bucket: host launch time, GPU time of the experts (split into jobs
    that found the GPU idle, "alone", and jobs queued behind another, "queued") and of the
    replies. CUDA-style events, read once completed, so timing adds no synchronization."""

    def __init__(self, keep: int = 4096):
        self.keep = keep
        self.pending = collections.deque()
        self.samples = collections.defaultdict(lambda: collections.defaultdict(list))

    def event(self, stream=None) -> torch.cuda.Event:
        e = torch.cuda.Event(enable_timing=True)
        e.record(stream)
        return e

    def start(self, stream=None) -> tuple:
        alone = not self.pending or self.pending[-1][4].query()
        return alone, self.event(stream)

    def add(self, n_tokens: int, started: tuple, experts, replied, host_s: float) -> None:
        bucket = 1 << (n_tokens - 1).bit_length()
        self.pending.append((bucket, *started, experts, replied, host_s))
        self.drain()

    def drain(self) -> None:
        while self.pending and self.pending[0][4].query():
            bucket, alone, start, experts, replied, host_s = self.pending.popleft()
            rows = self.samples[bucket]
            if len(rows["host_us"]) < self.keep:
                rows["host_us"].append(host_s * 1e6)
                rows["reply_ms"].append(experts.elapsed_time(replied))
                rows[f"experts_ms_{'alone' if alone else 'queued'}"].append(start.elapsed_time(experts))

    def summary(self) -> dict:
        torch.cuda.synchronize()
        self.drain()
        out = {}
        for bucket, rows in sorted(self.samples.items()):
            out[bucket] = {"jobs": len(rows["host_us"])}
            for name, values in sorted(rows.items()):
                out[bucket][f"{name}_p50"] = round(statistics.median(values), 4)
                out[bucket][f"{name}_n"] = len(values)
        return out


class FfnScheduler:
    """Serves the jobs an ``FfnServer`` discovers with the routed experts of every layer."""

    def __init__(self, server, experts: Dict[int, torch.nn.Module], *, graph_max_tokens: int = 0,
                 reply_stream: bool = True, timing: bool = False):
        self.server, self.g = server, server.g
        self.experts = experts
        first = next(iter(experts.values()))
        self.local = first.local
        self.stream = torch.cuda.Stream()
        self.reply_stream = torch.cuda.Stream() if reply_stream else None
        self.reply_ready = torch.cuda.Event()
        self.reply_free = [torch.cuda.Event(), torch.cuda.Event()]
        self.reply_turn = 0
        self.layer_calls: collections.Counter = collections.Counter()
        self.job_timer = JobTimer() if timing else None
        self.graph_runner: Optional[FfnGraphRunner] = None
        if graph_max_tokens:
            with torch.cuda.stream(self.stream):
                self.graph_runner = FfnGraphRunner(experts, graph_max_tokens, self.local, act=self.g.act)

    @torch.no_grad()
    def warmup(self, n_max: int) -> list:
        """Run every power-of-two token count up to n_max once (layer 0; every layer up to 256
        tokens), so every kernel and workspace is ready before serving."""
        layers = sorted(self.experts)
        first = self.experts[layers[0]]
        device = torch.cuda.current_device()
        buckets = graph_buckets(n_max)
        gen = torch.Generator(device=device).manual_seed(0)
        with torch.cuda.stream(self.stream):
            for n in buckets:
                x = torch.randn(n, first.hidden_size, device=device, dtype=torch.bfloat16, generator=gen)
                scores = torch.rand(n, first.num_experts, device=device, generator=gen)
                topk_ids = scores.topk(first.top_k, dim=1).indices.to(torch.int32)
                topk_weights = torch.rand(n, first.top_k, device=device, generator=gen)
                topk_output = StandardTopKOutput(topk_weights, topk_ids, None)
                for layer_id in layers[:1] if n > 256 else layers:
                    self.experts[layer_id](x, topk_output)
        torch.cuda.synchronize()
        return buckets

    def rows_of(self, row):
        """x, topk_ids and topk_weights of one row: views into the RecvArena. x is a tuple:
        (bf16 [n, H],) or, with fp8 activations on the wire, (e4m3 codes, scales)."""
        g, arena = self.g, self.server.recv
        n, off = row.n_tokens, row.x_ptr - self.server.recv_base
        if g.act == "bf16":
            x = (arena[off : off + n * g.hidden * 2].view(torch.bfloat16).view(n, g.hidden),)
        else:
            shape, dtype = act_scale_shape(g.act, n, g.hidden)
            xs_off = off + g.xs_off
            x = (arena[off : off + n * g.hidden].view(n, g.hidden),
                 arena[xs_off : xs_off + n * g.xs_bytes_per_token].view(dtype).view(shape))
        ids_off, w_off = off + g.ids_off, off + g.w_off
        topk_ids = arena[ids_off : ids_off + n * g.topk * 4].view(torch.int32).view(n, g.topk)
        topk_weights = arena[w_off : w_off + n * g.topk * 4].view(torch.float32).view(n, g.topk)
        return x, topk_ids, topk_weights

    @torch.no_grad()
    def run_job(self, job) -> None:
        """One expert call for the job's rows, then one reply per row. Only enqueues."""
        tic, timer = time.perf_counter(), self.job_timer
        stream = self.stream
        self.server.wait_rows(job, stream.cuda_stream)
        with torch.cuda.stream(stream):
            started = timer.start(stream) if timer else None
            rows = [self.rows_of(row) for row in job.rows]
            if len(rows) == 1:
                x, topk_ids, topk_weights = rows[0]
            else:
                x = tuple(torch.cat(part) for part in zip(*(r[0] for r in rows)))
                topk_ids, topk_weights = (torch.cat(part) for part in zip(*(r[1:] for r in rows)))
            n = topk_ids.shape[0]
            output, buffer, used_buffer = None, 0, False
            reply = self.reply_stream
            out = None
            if len(job.rows) == 1:  # write the partial sum straight into A's segment
                out = self.server.seg_view(job.rows[0])
            if self.graph_runner is not None and n <= self.graph_runner.buckets[-1]:
                if out is None and reply is not None:
                    buffer, used_buffer = self.reply_turn, True
                    # the reply that last read this buffer, before the replay overwrites it
                    stream.wait_event(self.reply_free[buffer])
                output = self.graph_runner.run(job.layer_id, x, topk_ids, topk_weights, buffer, out=out)
            if output is None:
                topk_output = StandardTopKOutput(topk_weights, topk_ids, None)
                layer = self.experts[job.layer_id]
                if len(x) == 1:
                    output = layer(x[0], topk_output, out=out)
                else:  # fp8 on the wire: the rows are quantized already
                    output = layer.forward_q(*x, topk_output, out=out)
            experts_done = timer.event(stream) if timer else None
        if reply is None:
            rstream = stream
        else:
            self.reply_ready.record(stream)
            reply.wait_event(self.reply_ready)
            rstream = reply
        start = 0
        for row in job.rows:
            nbytes = row.n_tokens * self.g.hidden * 2
            self.server.reply(row, output[start].data_ptr(), nbytes, rstream.cuda_stream)
            start += row.n_tokens
        self.layer_calls[job.layer_id] += 1
        if used_buffer:
            self.reply_free[buffer].record(reply)
            self.reply_turn = 1 - buffer
        if timer:
            timer.add(n, started, experts_done, timer.event(rstream), time.perf_counter() - tic)

    def serve_pending(self) -> int:
        """Poll once and run every complete job (the one-GPU form of serve_forever)."""
        return self.server.serve_pending(self.run_job)
