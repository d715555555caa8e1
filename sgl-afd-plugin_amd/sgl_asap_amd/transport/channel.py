"""A side of the transport on one MI355X: ``AttnChannel`` and its ``StallWatch``.

The attention rank's end of the connection to every F rank (the role of
``python/sgl_asap_plugin/transport/channel.py``): ``send`` enqueues one message of a slot
(the reference's :317-362) as one ``afd_send`` call, ``wait`` enqueues the waits for the F
ranks' answers (:364-377) as one ``afd_wait_replies`` call and returns the result segments,
``check`` raises ``ChannelPoisoned`` once a wait had to be released, and ``reconnect`` is the
way out (:301-311). ``_backpressure`` / ``_epoch_override`` are for tests that provoke
protocol violations (:198-203).

Design on one GPU:
* Every (F rank, slot) has a 64-bit done counter in a pinned host page. Message m of a slot
  has count ``base + m``; F's reply stores that count, A's streams wait for ``counter >= m``
  (backpressure before overwriting the slot's region: ``>= m - 1``). Counts only grow, so the
  32-bit sequence field of the doorbell word may wrap while no wait ever compares across it.
* The per-slot part of the send descriptor (regions, doorbell and counter addresses) is
  built once at connect; a send fills in the payload pointers, sizes and doorbell words and
  makes one C call, so the host enqueue of a message is a single ctypes call.
* Liveness: ``StallWatch`` reads the done counters straight from the pinned page. A counter
  that some stream waits on and that has not moved for ``timeout_s`` means the F side is dead
  or stuck; the watch then stores every awaited count (which releases every parked wait, the
  counters being compared with >=) and poisons the channel. It needs no events and no GPU
  calls, so a scan is a few loads.
"""

from __future__ import annotations

import threading
import time
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional, Sequence, Tuple

from .. import _lib
from . import hip
from .layout import ID_BYTES, ChannelPoisoned, Geometry, HandshakeError, pack_doorbell

COUNT_LIMIT = 1 << 63  # the largest base a channel accepts: counts never reach 2^64


def serve_before_waiting(servers: Sequence, a: int, slot: int, count: int, pump: Callable[[], object]) -> None:
    """Make sure an in-process F side has enqueued the job that answers message ``count`` of
    A rank ``a`` on ``slot`` before a stream is made to wait for that answer (the backpressure
    wait of the slot's next send, or the reply wait). Streams can share a hardware queue, and
    a wait enqueued ahead of the job that satisfies it then never ends.

    The message's word may still wait in an inbox, or its row in a half-formed job whose other
    rows' words are in an inbox: then ``pump`` (the F side's serve_pending) runs first. A row
    still half-formed after that needs rows that the other A ranks of its group have not sent,
    so no job can answer it yet and the wait is refused (RuntimeError) instead of enqueued."""
    states = [sv.pending_state(a, slot, count) for sv in servers]
    if "inbox" in states or ("forming" in states and any(sv.has_words() for sv in servers)):
        pump()
        states = [sv.pending_state(a, slot, count) for sv in servers]
    if "forming" in states:
        raise RuntimeError(
            f"A rank {a}: message #{count} on slot {slot} is waiting for the rows of its group's other A "
            "ranks; they must send before this rank waits for its answer (a stream parked on an answer "
            "that no enqueued job can give stalls the GPU queue it shares)"
        )


class StallWatch:
    """Detects a dead F side from the done counters an attention rank waits on.

    ``expect(offset, value, what)`` records that a stream will wait for the counter at
    ``offset`` of ``page`` to reach ``value``. ``scan(now)`` forgets satisfied expectations,
    restarts the quiet clock of every outstanding counter that moved, and if one has stayed
    unchanged for more than ``timeout_s`` stores every outstanding expected value (releasing
    all parked waits) and returns the description of the wait that stalled. ``start`` runs
    ``scan`` every ``period_s`` on a daemon thread and calls ``on_stall`` with the result."""

    def __init__(self, page, timeout_s: float, on_stall: Callable[[str], None], period_s: float = 0.02):
        self.page, self.timeout_s, self.on_stall, self.period_s = page, timeout_s, on_stall, period_s
        self._want: Dict[int, Tuple[int, str]] = {}  # offset -> (largest awaited value, its wait)
        self._quiet: Dict[int, Tuple[int, float]] = {}  # offset -> (value seen, since when)
        self._lock = threading.Lock()
        self._halt = threading.Event()
        self._thread: Optional[threading.Thread] = None

    def expect(self, offset: int, value: int, what: str) -> None:
        with self._lock:
            if value > self._want.get(offset, (-1, ""))[0]:
                self._want[offset] = (value, what)

    def outstanding(self) -> Dict[int, int]:
        with self._lock:
            return {off: v for off, (v, _) in self._want.items()}

    def scan(self, now: Optional[float] = None) -> Optional[str]:
        now = time.monotonic() if now is None else now
        with self._lock:
            stalled = None
            for off in list(self._want):
                value, what = self._want[off]
                seen = self.page.load(off)
                if seen >= value:
                    del self._want[off]
                    self._quiet.pop(off, None)
                    continue
                last = self._quiet.get(off)
                if last is None or last[0] != seen:
                    self._quiet[off] = (seen, now)
                elif now - last[1] > self.timeout_s and stalled is None:
                    stalled = what
            if stalled is None:
                return None
            for off, (value, _) in self._want.items():
                self.page.store(off, value)
            self._want.clear()
            self._quiet.clear()
            return stalled

    def _loop(self) -> None:
        while not self._halt.wait(self.period_s):
            what = self.scan()
            if what is not None:
                self.on_stall(what)

    def start(self) -> "StallWatch":
        self._thread = threading.Thread(target=self._loop, name="afd-stall-watch", daemon=True)
        self._thread.start()
        return self

    def stop(self) -> None:
        self._halt.set()
        if self._thread is not None and self._thread.is_alive():
            self._thread.join(timeout=5.0)
        self._thread = None


@dataclass(frozen=True)
class Ticket:
    """A sent message: its slot, its 64-bit count on that slot, and what it carried."""

    slot: int
    seq: int
    layer_id: int
    n_tokens: int


class AttnChannel:
    """A rank ``a``'s connection to every F rank (``servers[f]`` is F rank f's server)."""

    def __init__(self, a: int, geometry: Geometry, servers: Sequence, *, device: int = 0,
                 seq_base: int = 0, timeout_s: float = 60.0, _backpressure: bool = True,
                 _epoch_override: Optional[int] = None):
        if len(servers) != geometry.num_f:
            raise ValueError(f"need one server per F rank ({geometry.num_f}), got {len(servers)}")
        if not 0 <= a < geometry.num_a:
            raise ValueError(f"A rank {a} is outside [0, {geometry.num_a})")
        if geometry.num_f > _lib.AFD_MAX_F:
            raise ValueError(f"at most {_lib.AFD_MAX_F} F ranks, got {geometry.num_f}")
        if not 0 <= seq_base < COUNT_LIMIT:
            raise ValueError(f"seq_base must be in [0, 2^63), got {seq_base}")
        self.a, self.g, self.servers = a, geometry, list(servers)
        self.device, self.seq_base, self.timeout_s = device, seq_base, timeout_s
        self._backpressure, self._epoch_override = _backpressure, _epoch_override
        self.flags: Optional[hip.HostPage] = None
        self.segments = None  # device uint8 tensor: num_f * slots result segments
        self.watch: Optional[StallWatch] = None
        self._poison: Optional[ChannelPoisoned] = None
        # with the F rank in this process: its serve call (FfnScheduler.serve_pending), run by
        # send before a backpressure wait the host does not see satisfied yet
        self.pump: Optional[Callable[[], object]] = None
        self._count: List[int] = []
        self._epochs: List[int] = []
        self._desc: List[_lib.AfdSendDesc] = []
        self._done_addrs: List[List[int]] = []

    # ---- lifetime ----
    def connect(self) -> "AttnChannel":
        """Fresh done counters (all at seq_base) and result segments; one handshake per F
        rank; the per-slot send descriptors."""
        import torch

        g = self.g
        self.flags = hip.HostPage(g.flags_bytes)
        self.segments = torch.empty(g.num_f * g.slots * g.seg_bytes, dtype=torch.uint8,
                                    device=f"cuda:{self.device}")
        arenas, bells = [], []
        try:
            for f in range(g.num_f):
                for s in range(g.slots):
                    self.flags.store(g.done_off(f, s), self.seq_base)
            self._epochs = []
            for server in self.servers:
                answer = server.hello(self.a, self.flags, self.segments, g)
                if answer["seq_base"] != self.seq_base:
                    raise HandshakeError(f"seq_base A={self.seq_base} F={answer['seq_base']}")
                arenas.append(answer["recv"])
                bells.append(answer["doorbells"])
                self._epochs.append(answer["epoch"])
        except BaseException:
            self.close()
            raise
        self._desc, self._done_addrs = [], []
        for s in range(g.slots):
            d = _lib.AfdSendDesc()
            d.num_f = g.num_f
            d.xs_off, d.ids_off, d.w_off = g.xs_off, g.ids_off, g.w_off
            done = [self.flags.addr(g.done_off(f, s)) for f in range(g.num_f)]
            for f in range(g.num_f):
                d.region[f] = arenas[f] + g.region_off(self.a, s)
                d.bell[f] = bells[f].addr(g.bell_off(self.a, s))
                d.done[f] = done[f] if self._backpressure else None
            self._desc.append(d)
            self._done_addrs.append(done)
        self._count = [self.seq_base] * g.slots
        self._poison = None
        self.watch = StallWatch(self.flags, self.timeout_s, self._stalled).start()
        return self

    def reconnect(self) -> "AttnChannel":
        """Tear the channel down and connect again with fresh counters, segments and epochs;
        a channel whose wait was released stays unusable until this is called."""
        self.close()
        return self.connect()

    def close(self) -> None:
        """Stops the stall watch and frees the host pages and device segments; work still
        queued on a stream that uses them must have finished (synchronize it first)."""
        if self.watch is not None:
            self.watch.stop()
            self.watch = None
        if self.flags is not None:
            self.flags.release()
            self.flags = None
        self.segments = None
        self._desc, self._done_addrs = [], []

    def _stalled(self, what: str) -> None:
        self._poison = ChannelPoisoned(
            f"A rank {self.a}: {what} saw no answer for {self.timeout_s}s; the F side is dead or "
            "stuck, its pending waits were released and their results are invalid until reconnect()"
        )

    def check(self) -> None:
        """Raise ``ChannelPoisoned`` if a wait had to be released."""
        if self._poison is not None:
            raise self._poison

    # ---- addresses ----
    def seg_ptr(self, f: int, slot: int) -> int:
        return self.segments.data_ptr() + self.g.seg_off(f, slot) - self.g.flags_bytes

    def result_view(self, f: int, slot: int, n_tokens: int):
        """F rank f's partial sum for ``slot`` as it lies in this rank's result segment:
        bf16 [n_tokens, hidden] (valid after the wait for the reply, until the next reply)."""
        import torch

        off = self.g.seg_off(f, slot) - self.g.flags_bytes
        seg = self.segments[off : off + n_tokens * self.g.hidden * 2]
        return seg.view(torch.bfloat16).view(n_tokens, self.g.hidden)

    def done_count(self, f: int, slot: int) -> int:
        """The done counter of (F rank f, slot) as the host sees it now."""
        return self.flags.load(self.g.done_off(f, slot))

    # ---- messages ----
    def send(self, layer_id: int, slot: int, x_ptr: int, ids_ptr: int, w_ptr: int, n_tokens: int, stream,
             xs_ptr: int = 0) -> Ticket:
        """Enqueue one message on ``stream`` (a torch stream): ``n_tokens`` rows of x (bf16
        [n, hidden], or with fp8 activations on the wire the e4m3 codes [n, hidden] at x_ptr
        and their scales at xs_ptr), top-k ids (int32 [n, topk]) and weights (fp32 [n, topk])
        to every F rank."""
        self.check()
        g = self.g
        if not (0 <= slot < g.slots and 1 <= n_tokens <= g.n_max):
            raise ValueError(f"slot {slot} / n_tokens {n_tokens} outside the geometry {g}")
        if (g.act != "bf16") != bool(xs_ptr):
            raise ValueError(f"activation format {g.act} {'needs' if not xs_ptr else 'takes no'} scales")
        seq = self._count[slot] + 1
        d = self._desc[slot]
        d.x, d.x_bytes = x_ptr, n_tokens * g.x_bytes_per_token
        d.xs, d.xs_bytes = (xs_ptr or None), n_tokens * g.xs_bytes_per_token
        d.ids, d.w, d.ids_bytes = ids_ptr, w_ptr, n_tokens * g.topk * ID_BYTES
        d.done_min = seq - 1
        pending = False  # some F rank has not answered the slot's previous message yet
        for f in range(g.num_f):
            epoch = self._epochs[f] if self._epoch_override is None else self._epoch_override
            d.word[f] = pack_doorbell(seq, n_tokens, layer_id, epoch)
            if self._backpressure:
                # an answer the host already sees needs no wait on the GPU (the wait is a
                # kernel there, which may have to queue for a free CU)
                answered = self.flags.load(g.done_off(f, slot)) >= seq - 1
                d.done[f] = None if answered else self._done_addrs[slot][f]
                pending = pending or not answered
        if pending and self.pump is not None:
            # in-process F side: the job answering the slot's previous message must be enqueued
            # before this send's stream waits for the answer
            serve_before_waiting(self.servers, self.a, slot, seq - 1, self.pump)
        hip.send(d, stream.cuda_stream)
        self._count[slot] = seq
        for f, server in enumerate(self.servers):
            server.announce(self.a, slot, d.word[f])
        if pending:
            for f in range(g.num_f):
                self.watch.expect(g.done_off(f, slot), seq - 1, f"send of layer {layer_id} slot {slot} #{seq}")
        return Ticket(slot, seq, layer_id, n_tokens)

    def wait(self, ticket: Ticket, stream) -> List[int]:
        """Parks ``stream`` until each F rank's done counter for the ticket's slot reaches the
        ticket's sequence number, and gives back where those ranks' partial sums lie (one
        device address per F rank, in rank order, each bf16 [n_tokens, hidden])."""
        self.check()
        g, slot = self.g, ticket.slot
        if self.pump is not None and any(self.flags.load(g.done_off(f, slot)) < ticket.seq for f in range(g.num_f)):
            serve_before_waiting(self.servers, self.a, slot, ticket.seq, self.pump)
        hip.wait_replies(self._done_addrs[slot], ticket.seq, stream.cuda_stream)
        for f in range(g.num_f):
            self.watch.expect(g.done_off(f, slot), ticket.seq,
                              f"reply to layer {ticket.layer_id} slot {slot} #{ticket.seq}")
        return [self.seg_ptr(f, slot) for f in range(g.num_f)]
