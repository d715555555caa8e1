"""One attention rank and one FFN rank on one MI355X: the AFD loop of a single GPU.

Wires the pieces the reference runs in separate processes (``AsapBuffer.connect``,
``python/sgl_asap_plugin/srt/layers/moe/token_dispatcher/asap.py:99-147``;
``FfnScheduler.init_ffn_server``, ``srt/managers/scheduler.py:220-312``) into one process:

    AsapMoE.forward -> AsapDispatcher.dispatch -> AttnChannel.send   (A send stream)
        copies x / ids / w into the RecvArena, rings the doorbell
        pump: FfnServer.poll -> FfnScheduler.run_job                (F stream)
            gates on the doorbell, runs the experts into A's result segment, stores the
            message's count into A's done counter
    [shared experts on the compute stream]
    AsapDispatcher.combine -> AsapBuffer.recv
        pump again (serves whatever is still pending)
        AttnChannel.wait (compute stream: done counter >= count) -> afd_combine (+ shared)

Every wait is enqueued after the work that satisfies it (host order equals causal order),
so the loop cannot deadlock even when streams share a hardware queue.
"""

from __future__ import annotations

from typing import Dict, Optional

import torch

from .moe.dispatcher import AsapBuffer
from .runner.scheduler import FfnScheduler
from .transport.channel import AttnChannel
from .transport.layout import Geometry
from .transport.server import FfnServer


class OneGpuAfd:
    """``replicas`` x ``group`` A ranks (``group`` A ranks per replica, whose rows form one F
    job) and one F rank on one GPU. A rank 0's channel is installed as this process's
    ``AsapBuffer``; the others are driven through ``channels[a]`` directly (``AttnChannel.send`` / ``wait``, pump with ``serve_pending``).
    ``act``: the activation format on the wire ("bf16", or the experts' "mxfp8" /
    "fp8_1x128": A quantizes before the copy). ``f_streams``: the F streams eager jobs
    alternate over (default: replicas x slots, one per job that can be in flight).
    ``batch_tokens``: serve the bf16 jobs pending together in batched expert calls of up to
    that many tokens (0: one call per job)."""

    def __init__(self, experts: Dict[int, torch.nn.Module], *, n_max: int, slots: int = 2,
                 replicas: int = 1, group: int = 1, seq_base: int = 0, graph_max_tokens: int = 0,
                 timeout_s: float = 60.0, device: int = 0, act: str = "bf16",
                 timing: bool = False, f_streams: Optional[int] = None, batch_tokens: int = 0,
                 _backpressure: bool = True,
                 _epoch_override: Optional[int] = None):
        first = next(iter(experts.values()))
        if first.n_max < n_max:
            raise ValueError(f"experts hold workspaces for {first.n_max} tokens, the loop carries up to {n_max}")
        self.geometry = Geometry(num_a=replicas * group, group=group, slots=slots, n_max=n_max,
                                 hidden=first.hidden_size, topk=first.top_k, num_f=1, act=act)
        reads = {str(getattr(layer, "act_format", None)) for layer in experts.values()}
        if act != "bf16" and reads != {act}:
            raise ValueError(f"activations on the wire as {act}, but the experts read {sorted(reads)}")
        self.server = FfnServer(0, self.geometry, device=device, seq_base=seq_base).start()
        self.scheduler = FfnScheduler(self.server, experts, graph_max_tokens=graph_max_tokens, timing=timing,
                                      streams=f_streams, batch_tokens=batch_tokens)
        self.channels = [
            AttnChannel(a, self.geometry, [self.server], device=device, seq_base=seq_base,
                        timeout_s=timeout_s, _backpressure=_backpressure,
                        _epoch_override=_epoch_override).connect()
            for a in range(replicas * group)
        ]
        for channel in self.channels:
            channel.pump = self.scheduler.serve_pending
        self.channel = self.channels[0]
        self.buffer = AsapBuffer.install(self.channel, device, pump=self.scheduler.serve_pending)

    def close(self) -> None:
        torch.cuda.synchronize()
        if AsapBuffer._buffer is self.buffer:
            AsapBuffer.uninstall()
        for channel in self.channels:
            channel.close()
        self.server.close()

    def __enter__(self) -> "OneGpuAfd":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
