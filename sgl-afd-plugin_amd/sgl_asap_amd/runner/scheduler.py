"""The F rank's job handler: routed experts per MoE layer, served job by job.

Plays the part of ``FfnScheduler`` in ``python/sgl_asap_plugin/srt/managers/scheduler.py``:
``local_experts`` (:206-218), ``warmup`` (:329-351), ``run_job`` (:387-436), ``rows_of``
(:438-450) and the per-job timing of its ``JobTimer`` (:109-159).

Design on one GPU: everything a job does is stream-ordered on one F stream (jobs in turn over
one stream per job that can be in flight, so concurrent jobs overlap), enqueued by ``run_job``
without any host wait:

    gate on the rows' doorbells -> expert call -> reply (copies if any, then the done counters)

A job of one row (the normal case, one attention rank per replica) writes its output straight
into that rank's result segment, so its reply is only the done counter, which the eager expert
call stores itself (afd_moe_ffn_answer). The expert call is one C call that enqueues the whole
job (five launches); HIP graphs of it (``graph_max_tokens``, the reference runner's buckets)
are available, but on this stack a replay costs more host time (~60 vs ~35 µs per job) and
~14 µs more GPU time (a gap after each graph launch plus the descriptor write) than the eager
call, so the default is eager. A job of several rows
(a group of A ranks per replica) computes into a buffer that the reply copies from on the
same stream, so one output buffer is enough and its memory is never handed out while a copy
still reads it. With fp8 activations on the wire (``Geometry.act``) the rows arrive as e4m3
codes plus scales and the expert call runs on them as they are.

Batching (``batch_tokens`` > 0; the reference runs one expert call per job): the single-row
jobs of one poll that belong to the same layer are packed, largest first, into batches
of at most ``batch_tokens`` tokens and AFD_MAX_BATCH jobs, each served by one expert call
(afd_moe_ffn_batch) on one F stream after gating on every job's doorbell. Every job still gets
its own output in its A rank's segment and its own done counter, and its output is the same
bit for bit as when served alone; the batch streams each expert's weights once for all its
jobs and fills their row tiles together.
"""

from __future__ import annotations

import collections
import time
from typing import Dict, List, Optional

import numpy as np
import torch

from .. import _lib
from ..moe.experts import act_scale_shape
from ..moe.topk import StandardTopKOutput
from .graph_runner import FfnGraphRunner, graph_buckets


def local_experts(ep_rank: int, ep_size: int, num_experts: int) -> range:
    """The routed experts of EP rank ``ep_rank``: a contiguous block of num_experts // ep_size
    global ids."""
    width = num_experts // ep_size
    return range(ep_rank * width, ep_rank * width + width)


class JobClock:
    """GPU and host time of every served job, grouped by the job's power-of-two size class.

    ``start`` / ``stop`` bracket a job's GPU work with two timing events on the job's F stream
    and note the host time spent enqueueing it; whether that stream was idle when the job was
    enqueued is recorded too (the end event of the stream's previous job had completed), since
    a job queued behind another starts late. Records are resolved lazily: ``collect`` reads only those
    whose end event the GPU has passed, so timing never synchronizes the serving loop."""

    def __init__(self, keep: int = 4096):
        self.keep = keep
        self._open: collections.deque = collections.deque()
        self._rows: Dict[int, List[tuple]] = collections.defaultdict(list)
        self._last_end: Dict[int, torch.cuda.Event] = {}  # per F stream

    @staticmethod
    def size_class(n_tokens: int) -> int:
        return 1 << max(0, n_tokens - 1).bit_length()

    def start(self, stream) -> tuple:
        last = self._last_end.get(stream.cuda_stream)
        idle = last is None or last.query()
        begin = torch.cuda.Event(enable_timing=True)
        begin.record(stream)
        return time.perf_counter(), idle, begin

    def stop(self, token: tuple, n_tokens: int, stream) -> None:
        t0, idle, begin = token
        end = torch.cuda.Event(enable_timing=True)
        end.record(stream)
        self._last_end[stream.cuda_stream] = end
        self._open.append((self.size_class(n_tokens), idle, begin, end, time.perf_counter() - t0))
        self.collect()

    def collect(self) -> None:
        while self._open and self._open[0][3].query():
            size, idle, begin, end, host_s = self._open.popleft()
            rows = self._rows[size]
            if len(rows) < self.keep:
                rows.append((begin.elapsed_time(end), host_s * 1e6, idle))

    def summary(self) -> dict:
        """Per size class: job count, median / p90 GPU ms (split by whether the stream was
        idle at enqueue) and median host enqueue µs. Synchronizes the device first."""
        torch.cuda.synchronize()
        self.collect()
        out = {}
        for size in sorted(self._rows):
            gpu, host, idle = (np.asarray(c) for c in zip(*self._rows[size]))
            entry = {"jobs": int(gpu.size), "host_us_p50": round(float(np.median(host)), 2)}
            for name, sel in (("idle", idle), ("queued", ~idle)):
                if sel.any():
                    entry[f"gpu_ms_{name}_p50"] = round(float(np.median(gpu[sel])), 4)
                    entry[f"gpu_ms_{name}_p90"] = round(float(np.percentile(gpu[sel], 90)), 4)
                    entry[f"gpu_ms_{name}_n"] = int(sel.sum())
            out[size] = entry
        return out


class FfnScheduler:
    """Serves the jobs an ``FfnServer`` discovers with the routed experts of every layer."""

    def __init__(self, server, experts: Dict[int, torch.nn.Module], *, graph_max_tokens: int = 0,
                 timing: bool = False, streams: Optional[int] = None, batch_tokens: int = 0):
        self.server, self.g = server, server.g
        if batch_tokens < 0:
            raise ValueError(f"batch_tokens must be >= 0, got {batch_tokens}")
        self.batch_tokens = batch_tokens
        self.batch_calls = 0  # expert calls that served more than one job
        self.expert_calls = 0  # expert calls (or graph replays) of any kind
        self.experts = experts
        self.local = next(iter(experts.values())).local
        # A serving GPU is shared: the attention side's kernels and its parked stream waits
        # (a wait is a kernel on this stack) may hold CUs while a job runs, so the GEMMs take
        # their tiles dynamically (identical results; a static share would leave a whole round
        # to a workgroup that starts late).
        for layer in experts.values():
            layer.tile_walk = "dynamic"
        # Jobs go to ``streams`` F streams in turn (each with its own workspace, and with
        # graphs its own graph runner: workspace, descriptor and output buffers): jobs in
        # flight together run concurrently, each one's GEMMs taking the CUs that the others'
        # partial last rounds leave idle (results are the same; the dynamic tile walk lets a
        # late workgroup take fewer tiles). Default: one stream per job that can be in flight
        # at once, replicas x slots.
        if streams is None:
            streams = max(1, self.g.num_a // self.g.group) * self.g.slots
        if streams < 1:
            raise ValueError(f"streams must be >= 1, got {streams}")
        self.streams = [torch.cuda.Stream() for _ in range(streams)]
        self.stream = self.streams[0]
        self._turn = 0
        self.layer_calls: collections.Counter = collections.Counter()
        self.clock = JobClock() if timing else None
        self.graph_runners: List[FfnGraphRunner] = []
        if graph_max_tokens:
            for s in self.streams:
                with torch.cuda.stream(s):
                    self.graph_runners.append(
                        FfnGraphRunner(experts, graph_max_tokens, self.local, act=self.g.act))
        self.graph_runner: Optional[FfnGraphRunner] = self.graph_runners[0] if self.graph_runners else None

    @torch.no_grad()
    def warmup(self, n_max: int) -> list:
        """Run the expert call once at every graph-bucket size up to ``n_max`` on seeded
        inputs (the prefixes of one batch: x ~ N(0,1) bf16, k distinct experts per token drawn
        uniformly over all experts, weights ~ U(0,1)), on the first layer at every size and on
        every other layer at the smallest size, on the first F stream; on every other F stream
        each layer at the smallest size. So every kernel and every workspace has been used
        before serving; with ``batch_tokens``, also a batched call on every F stream (its
        workspace). Synchronizes; returns the sizes run."""
        order = sorted(self.experts)
        first = self.experts[order[0]]
        sizes = graph_buckets(n_max)
        device = torch.device("cuda", torch.cuda.current_device())
        gen = torch.Generator(device=device).manual_seed(0)
        n = sizes[-1]
        x = torch.randn(n, first.hidden_size, generator=gen, device=device).to(torch.bfloat16)
        ids = torch.multinomial(torch.ones(n, first.num_experts, device=device), first.top_k,
                                replacement=False, generator=gen).to(torch.int32)
        w = torch.rand(n, first.top_k, generator=gen, device=device)
        for stream in self.streams:  # the inputs come from the current stream
            stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            for i, size in enumerate(sizes):
                topk = StandardTopKOutput(w[:size], ids[:size])
                for layer_id in (order if i == 0 else order[:1]):
                    self.experts[layer_id](x[:size], topk)
        topk = StandardTopKOutput(w[: sizes[0]], ids[: sizes[0]])
        for stream in self.streams[1:]:
            with torch.cuda.stream(stream):
                for layer_id in order:
                    self.experts[layer_id](x[: sizes[0]], topk)
        if self.batch_tokens:
            # the batched calls' workspaces (one per F stream, batch_tokens tokens) are made now,
            # not by the first batch while serving: a batch of two one-token jobs on each stream
            out = torch.empty(2, first.hidden_size, dtype=torch.bfloat16, device=device)
            rows = [(1, x[i].data_ptr(), 0, ids[i].data_ptr(), w[i].data_ptr(), out[i].data_ptr(), 0, 0)
                    for i in range(2)]
            for stream in self.streams:
                with torch.cuda.stream(stream):
                    for layer_id in order:
                        self.experts[layer_id].call_batch_ptrs(rows, stream.cuda_stream, capacity=self.batch_tokens)
        torch.cuda.synchronize()
        return sizes

    def rows_of(self, row):
        """The arrived message of one row as tensors over the receive arena, without copying:
        (activations, ids int32 [n, k], weights fp32 [n, k]); the activations are a tuple,
        (bf16 [n, H],) or with fp8 on the wire (e4m3 codes, their scales)."""
        g, arena = self.g, self.server.recv
        n, base = row.n_tokens, row.x_ptr - self.server.recv_base

        def view(off, nbytes, dtype, shape):
            return arena[off : off + nbytes].view(dtype).view(shape)

        if g.act == "bf16":
            x = (view(base, n * g.hidden * 2, torch.bfloat16, (n, g.hidden)),)
        else:
            shape, dtype = act_scale_shape(g.act, n, g.hidden)
            x = (view(base, n * g.hidden, torch.uint8, (n, g.hidden)),
                 view(base + g.xs_off, n * g.xs_bytes_per_token, dtype, shape))
        topk_ids = view(base + g.ids_off, n * g.topk * 4, torch.int32, (n, g.topk))
        topk_weights = view(base + g.w_off, n * g.topk * 4, torch.float32, (n, g.topk))
        return x, topk_ids, topk_weights

    def _inputs(self, job):
        parts = [self.rows_of(row) for row in job.rows]
        if len(parts) == 1:
            return parts[0]
        x = tuple(torch.cat([p[0][i] for p in parts]) for i in range(len(parts[0][0])))
        return x, torch.cat([p[1] for p in parts]), torch.cat([p[2] for p in parts])

    def _experts(self, layer_id: int, x: tuple, ids, w, out, runner=None):
        if runner is not None:
            result = runner.run(layer_id, x, ids, w, 0, out=out)
            if result is not None:
                return result
        layer = self.experts[layer_id]
        topk = StandardTopKOutput(w, ids)
        return layer(x[0], topk, out=out) if len(x) == 1 else layer.forward_q(*x, topk, out=out)

    def _run_row(self, job, stream, runner) -> int:
        """A job of one row (one A rank per replica): the expert call reads the arena record
        and writes A's result segment through raw pointers, so no tensor is made on the way.
        The eager call also stores the reply (its last workgroup writes A's done counter once
        the output is visible), so the F stream needs no separate reply launch, which would
        queue behind whatever occupies the CUs; a graph replay is answered by ``reply_job``.
        Returns n."""
        row, g = job.rows[0], self.g
        n = row.n_tokens
        xs_ptr = row.x_ptr + g.xs_off if g.act != "bf16" else 0
        out_ptr = self.server.seg_ptr(row)
        if runner is not None:
            with torch.cuda.stream(stream):  # a replay runs on the current stream
                replayed = runner.run_ptrs(job.layer_id, n, row.x_ptr, xs_ptr, row.ids_ptr, row.w_ptr, out_ptr)
            if replayed:
                self.server.reply_job(job, out_ptr, stream.cuda_stream)
                return n
        self.experts[job.layer_id].call_ptrs(n, row.x_ptr, xs_ptr, row.ids_ptr, row.w_ptr, out_ptr,
                                             stream.cuda_stream, self.server.done_addr(row), row.seq)
        return n

    def _run_rows(self, job, stream, runner) -> int:
        """A job of several rows: their records concatenated, the output in a buffer that the
        reply copies into each A rank's segment (same stream, so the buffer is free again
        before the next job writes it). Returns n."""
        x, ids, w = self._inputs(job)
        output = self._experts(job.layer_id, x, ids, w, None, runner)
        self.server.reply_job(job, output.data_ptr(), stream.cuda_stream)
        return ids.shape[0]

    @torch.no_grad()
    def run_job(self, job) -> None:
        """Gate, expert call and reply of one job, all enqueued on one F stream (the next in
        turn)."""
        turn, stream = self._next_stream()
        runner = self.graph_runners[turn] if self.graph_runners else None
        self.server.gate(job, stream.cuda_stream)
        token = self.clock.start(stream) if self.clock is not None else None
        if len(job.rows) == 1:
            n = self._run_row(job, stream, runner)  # raw pointers on the F stream: no torch op
        else:
            with torch.cuda.stream(stream):
                n = self._run_rows(job, stream, runner)
        self.layer_calls[job.layer_id] += 1
        self.expert_calls += 1
        if token is not None:
            self.clock.stop(token, n, stream)

    def _next_stream(self):
        turn = self._turn
        self._turn = (turn + 1) % len(self.streams)
        return turn, self.streams[turn]

    def _batchable(self, job) -> bool:
        return len(job.rows) == 1 and job.rows[0].n_tokens <= self.batch_tokens

    @staticmethod
    def _generations(jobs) -> List[list]:
        """The jobs of one poll by generation: generation g holds the g-th job of each (replica,
        slot) of the poll, in arrival order. A slot's next message is rung only after the F side
        answered the one before, so the later job's doorbell gate must not be enqueued ahead of,
        or in the same batched call as, the earlier job's answer: the scheduler serves the
        generations one after another, and a batch holds jobs of one generation only."""
        seen: collections.Counter = collections.Counter()
        gens: List[list] = []
        for job in jobs:
            key = (job.replica, job.slot)
            gen = seen[key]
            seen[key] += 1
            if gen == len(gens):
                gens.append([])
            gens[gen].append(job)
        return gens

    def _pack(self, jobs) -> List[list]:
        """First-fit decreasing: jobs of one layer and one generation (at most one per
        (replica, slot)) into batches of at most batch_tokens tokens and AFD_MAX_BATCH jobs."""
        keys = [(job.replica, job.slot) for job in jobs]
        if len(set(keys)) != len(keys):
            raise ValueError("jobs to pack hold two messages of one (replica, slot); pack each generation apart")
        bins: List[list] = []
        room: List[int] = []
        for job in sorted(jobs, key=lambda j: -j.rows[0].n_tokens):
            n = job.rows[0].n_tokens
            for b, free in enumerate(room):
                if n <= free and len(bins[b]) < _lib.AFD_MAX_BATCH:
                    bins[b].append(job)
                    room[b] = free - n
                    break
            else:
                bins.append([job])
                room.append(self.batch_tokens - n)
        return bins

    @torch.no_grad()
    def run_batch(self, jobs) -> None:
        """Gates, one expert call and the replies of several single-row jobs of one layer,
        all on one F stream (the next in turn); a batch of one is ``run_job``."""
        if len(jobs) == 1:
            self.run_job(jobs[0])
            return
        layer_id = jobs[0].layer_id
        if any(job.layer_id != layer_id or not self._batchable(job) for job in jobs):
            raise ValueError("a batch holds single-row jobs of one layer within batch_tokens")
        if len({(job.replica, job.slot) for job in jobs}) != len(jobs):
            # the later message's gate would wait, ahead of the call, for a doorbell that is rung
            # only after the call answers the earlier one
            raise ValueError("a batch cannot hold two messages of one (replica, slot)")
        _, stream = self._next_stream()
        rows = []
        for job in jobs:
            self.server.gate(job, stream.cuda_stream)
            row = job.rows[0]
            xs_ptr = row.x_ptr + self.g.xs_off if self.g.act != "bf16" else 0
            rows.append((row.n_tokens, row.x_ptr, xs_ptr, row.ids_ptr, row.w_ptr, self.server.seg_ptr(row),
                         self.server.done_addr(row), row.seq))
        token = self.clock.start(stream) if self.clock is not None else None
        self.experts[layer_id].call_batch_ptrs(rows, stream.cuda_stream, capacity=self.batch_tokens)
        self.layer_calls[layer_id] += len(jobs)
        self.batch_calls += 1
        self.expert_calls += 1
        if token is not None:
            self.clock.stop(token, sum(r[0] for r in rows), stream)

    def serve_pending(self) -> int:
        """Poll once and run every complete job (the one-GPU form of serve_forever); with
        ``batch_tokens``, the batchable jobs of the poll in batches per layer."""
        if not self.batch_tokens:
            return self.server.serve_pending(self.run_job)
        jobs = self.server.poll()
        for generation in self._generations(jobs):
            by_layer: Dict[int, list] = collections.defaultdict(list)
            for job in generation:
                if self._batchable(job):
                    by_layer[job.layer_id].append(job)
                else:
                    self.run_job(job)
            for layer_jobs in by_layer.values():
                for batch in self._pack(layer_jobs):
                    self.run_batch(batch)
        return len(jobs)
