"""A side of the transport on one MI355X: ``AttnChannel`` and its ``Watchdog``.

Follows ``python/sgl_asap_plugin/transport/channel.py``: ``send`` (:317-362) enqueues, on
the caller's stream, the backpressure waits on every F rank's done flag, the three payload
copies into the F rank's RecvArena region and the 64-bit doorbell; ``wait`` (:364-377)
enqueues the waits for the replies and returns the result segment addresses; a
``Watchdog`` (:100-167) times the oldest unfinished group of waits and, on timeout, writes
every awaited value so the parked streams are released, after which ``check``/``send``
raise ``ChannelPoisoned`` until ``reconnect``. ``_backpressure`` / ``_epoch_override``
exist, as in the reference (:198-203), only for tests that provoke protocol violations.

On one GPU the done flags live in pinned host memory (``hip.HostPage``) rather than in
the ResultArena's device flag page, so the watchdog releases a parked wait with a plain
host store, independent of any GPU queue; the segments stay in device memory at the
reference's offsets (``Geometry.seg_off`` minus the flag page).
"""

from __future__ import annotations

import collections
import threading
import time
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence, Tuple

from . import hip
from .layout import (
    ID_BYTES,
    SEQ_MASK,
    ChannelPoisoned,
    Geometry,
    HandshakeError,
    pack_doorbell,
)


class _Phase:
    """A group of stream waits plus the event recorded right after them; ``release`` lists
    (page, offset, value) stores that satisfy every wait of the group."""

    __slots__ = ("event", "release", "what", "state", "t_head")

    def __init__(self, event, release: List[Tuple[hip.HostPage, int, int]], what: str):
        self.event, self.release, self.what = event, release, what
        self.state = "pending"
        self.t_head: Optional[float] = None


class Watchdog(threading.Thread):
    """Releases A's stream waits when F does not answer within ``timeout_s``.

    Phases of one stream finish in order, so only the oldest unfinished phase is timed, from
    when it became the oldest (an O(1) scan every ``SCAN_S``). On timeout every pending
    phase's awaited values are stored into the pinned flag pages, which releases all parked
    waits, and ``on_timeout`` is called."""

    SCAN_S = 0.02

    def __init__(self, timeout_s: float, on_timeout: Callable[[_Phase], None]):
        super().__init__(name="asap-watchdog", daemon=True)
        self.timeout_s, self.on_timeout = timeout_s, on_timeout
        self._queue: collections.deque = collections.deque()
        self._lock = threading.Lock()
        self._stop_evt = threading.Event()

    def watch(self, stream, release: List[Tuple[hip.HostPage, int, int]], what: str) -> _Phase:
        import torch

        event = torch.cuda.Event()
        event.record(stream)
        phase = _Phase(event, release, what)
        with self._lock:
            self._queue.append(phase)
        return phase

    def scan(self, now: Optional[float] = None) -> Optional[_Phase]:
        """One scan; returns the phase that timed out, if any."""
        now = time.monotonic() if now is None else now
        with self._lock:
            while self._queue and self._queue[0].event.query():
                done = self._queue.popleft()
                if done.state == "pending":
                    done.state = "done"
            head = self._queue[0] if self._queue else None
            if head is None or head.state != "pending":
                return None
            if head.t_head is None:
                head.t_head = now
                return None
            if now - head.t_head <= self.timeout_s:
                return None
            for p in self._queue:
                if p.state == "pending":
                    p.state = "failed"
                    for page, off, value in p.release:
                        page.store(off, value)
        return head

    def run(self) -> None:
        while not self._stop_evt.wait(self.SCAN_S):
            late = self.scan()
            if late is not None:
                self.on_timeout(late)

    def stop(self) -> None:
        self._stop_evt.set()
        if self.is_alive():
            self.join(timeout=5.0)
        with self._lock:
            self._queue.clear()


@dataclass
class Ticket:
    """One message in flight; ``send`` / ``reply`` are the watched phases of its waits."""

    slot: int
    seq: int
    layer_id: int
    n_tokens: int
    send: Optional[_Phase] = None
    reply: Optional[_Phase] = None
    result_ptrs: List[int] = field(default_factory=list)


class AttnChannel:
    """A rank ``a``'s connection to every F rank (``servers[f]`` is F rank f's server)."""

    def __init__(self, a: int, geometry: Geometry, servers: Sequence, *, device: int = 0,
                 seq_base: int = 0, timeout_s: float = 60.0, _backpressure: bool = True,
                 _epoch_override: Optional[int] = None):
        if len(servers) != geometry.num_f:
            raise ValueError(f"need one server per F rank ({geometry.num_f}), got {len(servers)}")
        if not 0 <= a < geometry.num_a:
            raise ValueError(f"A rank {a} is outside [0, {geometry.num_a})")
        self.a, self.g, self.servers = a, geometry, list(servers)
        self.device, self.seq_base, self.timeout_s = device, seq_base & SEQ_MASK, timeout_s
        self._backpressure, self._epoch_override = _backpressure, _epoch_override
        self._poison: Optional[ChannelPoisoned] = None
        self._watchdog: Optional[Watchdog] = None
        self.flags: Optional[hip.HostPage] = None
        self.segments = None  # device tensor of num_f * slots result segments
        self._recv: List[int] = []
        self._bells: List[hip.HostPage] = []
        self._epoch: List[int] = []
        self._seq: List[int] = []

    def connect(self) -> "AttnChannel":
        """Allocate the result flags and segments, hand them to every F rank, map their
        RecvArenas and doorbell pages."""
        import torch

        g = self.g
        self.flags = hip.HostPage(g.flags_bytes)
        for f in range(g.num_f):
            for s in range(g.slots):
                self.flags.store(g.done_off(f, s), self.seq_base)
        self.segments = torch.empty(g.num_f * g.slots * g.seg_bytes, dtype=torch.uint8, device=f"cuda:{self.device}")
        try:
            for server in self.servers:
                reply = server.hello(self.a, self.flags, self.segments, g)
                if reply["seq_base"] != self.seq_base:
                    raise HandshakeError(f"seq_base A={self.seq_base} F={reply['seq_base']}")
                self._recv.append(reply["recv"])
                self._bells.append(reply["doorbells"])
                self._epoch.append(reply["epoch"])
        except BaseException:
            self.close()
            raise
        self._seq = [self.seq_base] * g.slots
        self._poison = None
        self._watchdog = Watchdog(self.timeout_s, self._on_timeout)
        self._watchdog.start()
        return self

    def reconnect(self) -> "AttnChannel":
        """The only way out of a poisoned channel: fresh flags and segments, a new epoch."""
        self.close()
        return self.connect()

    def close(self) -> None:
        """Release everything (synchronize the streams that used the channel first)."""
        if self._watchdog is not None:
            self._watchdog.stop()
            self._watchdog = None
        if self.flags is not None:
            self.flags.release()
            self.flags = None
        self.segments = None
        self._recv, self._bells, self._epoch = [], [], []

    def _on_timeout(self, phase: _Phase) -> None:
        self._poison = ChannelPoisoned(
            f"A rank {self.a}: {phase.what} did not complete within {self.timeout_s}s, F is dead or stuck; "
            "the results of every pending message are garbage until reconnect()"
        )

    def check(self) -> None:
        if self._poison is not None:
            raise self._poison

    def done_offset(self, f: int, slot: int) -> int:
        return self.g.done_off(f, slot)

    def seg_ptr(self, f: int, slot: int) -> int:
        return self.segments.data_ptr() + self.g.seg_off(f, slot) - self.g.flags_bytes

    def result_view(self, f: int, slot: int, n_tokens: int):
        """F rank f's partial sum for ``slot`` as it lies in this rank's result segment:
        bf16 [n_tokens, hidden] (valid after the wait for the reply, until the next reply)."""
        import torch

        off = self.g.seg_off(f, slot) - self.g.flags_bytes
        seg = self.segments[off : off + n_tokens * self.g.hidden * 2]
        return seg.view(torch.bfloat16).view(n_tokens, self.g.hidden)

    def send(self, layer_id: int, slot: int, x_ptr: int, ids_ptr: int, w_ptr: int, n_tokens: int, stream,
             xs_ptr: int = 0) -> Ticket:
        """Enqueue one message on ``stream`` (a torch stream): ``n_tokens`` rows of x (bf16
        [n, hidden]), top-k ids (int32 [n, topk]) and weights (fp32 [n, topk]) to every F rank.
        With fp8 activations on the wire (``g.act`` != "bf16") x_ptr holds the e4m3 codes
        [n, hidden] and xs_ptr their scales [n, g.xs_bytes_per_token bytes]."""
        self.check()
        g = self.g
        if not (0 <= slot < g.slots and 1 <= n_tokens <= g.n_max):
            raise ValueError(f"slot {slot} / n_tokens {n_tokens} outside the geometry {g}")
        if (g.act != "bf16") != bool(xs_ptr):
            raise ValueError(f"activation format {g.act} {'needs' if xs_ptr == 0 else 'takes no'} scales")
        seq = self._seq[slot] = (self._seq[slot] + 1) & SEQ_MASK
        sh = stream.cuda_stream
        x_n, k_n = n_tokens * g.x_bytes_per_token, n_tokens * g.topk * ID_BYTES
        xs_n = n_tokens * g.xs_bytes_per_token
        if self._backpressure:  # the previous message of this slot must be answered first
            for f in range(g.num_f):
                hip.wait64(sh, self.flags.addr(g.done_off(f, slot)), (seq - 1) & SEQ_MASK)
        for f, server in enumerate(self.servers):
            epoch = self._epoch[f] if self._epoch_override is None else self._epoch_override
            dst = self._recv[f] + g.region_off(self.a, slot)
            hip.copy_async(dst, x_ptr, x_n, sh)
            if xs_n:
                hip.copy_async(dst + g.xs_off, xs_ptr, xs_n, sh)
            hip.copy_async(dst + g.ids_off, ids_ptr, k_n, sh)
            hip.copy_async(dst + g.w_off, w_ptr, k_n, sh)  # fp32 weights: the size of the int32 ids
            word = pack_doorbell(seq, n_tokens, layer_id, epoch)
            # the doorbell goes last in the same stream: F's wait on it implies the payload landed
            hip.write64(sh, self._bells[f].addr(g.bell_off(self.a, slot)), word)
            server.announce(self.a, slot, word)
        ticket = Ticket(slot, seq, layer_id, n_tokens)
        ticket.send = self._watchdog.watch(
            stream,
            [(self.flags, g.done_off(f, slot), (seq - 1) & SEQ_MASK) for f in range(g.num_f)],
            f"send of layer {layer_id} slot {slot} seq {seq}",
        )
        return ticket

    def wait(self, ticket: Ticket, stream) -> List[int]:
        """Enqueue on ``stream`` the waits for every F rank's answer to ``ticket``; returns the
        device addresses of the E partial sums (bf16 [n_tokens, hidden] each)."""
        self.check()
        g, slot, seq = self.g, ticket.slot, ticket.seq
        for f in range(g.num_f):
            hip.wait64(stream.cuda_stream, self.flags.addr(g.done_off(f, slot)), seq)
        ticket.reply = self._watchdog.watch(
            stream,
            [(self.flags, g.done_off(f, slot), seq) for f in range(g.num_f)],
            f"reply to layer {ticket.layer_id} slot {slot} seq {seq}",
        )
        ticket.result_ptrs = [self.seg_ptr(f, slot) for f in range(g.num_f)]
        return ticket.result_ptrs
