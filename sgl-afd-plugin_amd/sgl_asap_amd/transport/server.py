"""F side of the transport on one MI355X: the RecvArena, the doorbell page, job discovery,
the doorbell gate and the replies.

The F rank's end of the connection (the role of ``python/sgl_asap_plugin/transport/server.py``):
``hello`` admits an A rank and hands out its epoch (``(old % 31) + 1``, :237), discovery turns
doorbell words into ``Row`` / ``Job`` records (:47-81) under the reference's rules, and
``reply_job`` answers a job (:340-350) with one ``afd_reply`` call (or, for a job whose output
the expert call writes in place, ``done_addr`` hands the counter to that call, which stores it
itself).

Discovery, on one GPU: A's producer stream rings the doorbell in pinned host memory with a
64-bit stream store, and ``AttnChannel.send`` also posts the same word to ``announce``. The
server keeps the posted words in one arrival-ordered inbox, so its host learns of a message
the moment it is enqueued, without waiting for the GPU, and ``gate`` then parks the F stream
on the real doorbell so the experts start once the payload has landed. Because every posted
word stays in the inbox until a poll consumes it, a message is never overwritten unread (two
sends on one slot before a poll are served in order), and jobs are handed out first come,
first served across A ranks.

Rules a word is checked against, in this order (the reference's, with its stats keys):
* sequence: the word's 32-bit sequence field against the last one seen on its (a, slot),
  as a cyclic int32 difference; 0 or negative -> an old word, ignored; d > 1 -> d - 1
  messages were never posted (``lost_messages``); the 64-bit count of the message is the
  last count + d;
* the A rank must have said hello (``unknown_peer``), the word must carry its current epoch
  (``stale_epoch``), and 1 <= n_tokens <= n_max (``bad_doorbell``);
* the rows of one replica's group of A ranks (``Geometry.group``) for one slot form a job once
  all have arrived; they must name the same layer (``group_mismatch``).
Handshakes are calls (``hello``) instead of a TCP JSON line: A and F share a process.
"""

from __future__ import annotations

import collections
import ctypes
import time
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional

from .. import _lib
from . import hip
from .layout import MAX_EPOCH, SEQ_MASK, Geometry, HandshakeError, seq_ahead, unpack_doorbell


@dataclass
class Peer:
    """A connected A rank: its done-counter page, its result segments and its epoch."""

    a: int
    flags: Optional[hip.HostPage]
    segments: object  # device uint8 tensor: the rank's result segments (at seg_off - flags_bytes)
    epoch: int


@dataclass
class Row:
    """One A rank's part of a job. ``seq`` is the message's 64-bit count on its slot; the
    pointers address this F rank's RecvArena."""

    a: int
    slot: int
    seq: int
    epoch: int
    layer_id: int
    n_tokens: int
    x_ptr: int
    ids_ptr: int
    w_ptr: int


@dataclass
class Job:
    """One micro-batch of one layer of one replica, ready to compute (rows in group order)."""

    replica: int
    slot: int
    layer_id: int
    rows: List[Row]
    t_detect_ns: int


class FfnServer:
    """One F rank's end of the transport: ``start`` -> ``hello`` per A rank -> ``poll`` /
    ``serve_pending`` -> ``gate`` + ``reply_job`` -> ``close``.

    ``memory="none"`` skips the device and pinned allocations (host-logic tests)."""

    STATS = ("lost_messages", "unknown_peer", "stale_epoch", "bad_doorbell", "group_mismatch", "jobs",
             "replica_switches", "reconnects", "dropped_replies")

    def __init__(self, f_rank: int, geometry: Geometry, *, device: int = 0, seq_base: int = 0,
                 memory: str = "device", trace_len: int = 4096):
        if memory not in ("device", "none"):
            raise ValueError(f"memory must be 'device' or 'none', got {memory!r}")
        self.f, self.g, self.seq_base = f_rank, geometry, seq_base
        self.device, self.memory = device, memory
        self.stats: collections.Counter = collections.Counter({k: 0 for k in self.STATS})
        self.trace: collections.deque = collections.deque(maxlen=trace_len)
        self.peers: Dict[int, Peer] = {}
        self.recv = None
        self.recv_base = 0
        self.bells: Optional[hip.HostPage] = None
        self._inbox: collections.deque = collections.deque()  # (a, slot, word) in arrival order
        self._count: List[int] = []  # per (a, slot): 64-bit count of the last word taken
        self._forming: Dict[tuple, Dict[int, Row]] = {}  # (replica, slot) -> rows so far
        self._last_replica: Optional[int] = None

    # ---- lifetime ----
    def start(self) -> "FfnServer":
        """Allocate the RecvArena (device) and the doorbell page (pinned host); every doorbell
        holds seq_base."""
        g = self.g
        if self.memory == "device":
            import torch

            self.recv = torch.zeros(g.recv_bytes, dtype=torch.uint8, device=f"cuda:{self.device}")
            self.recv_base = self.recv.data_ptr()
            self.bells = hip.HostPage(g.host_bytes)
            for a in range(g.num_a):
                for s in range(g.slots):
                    self.bells.store(g.bell_off(a, s), self.seq_base & SEQ_MASK)
        self._count = [self.seq_base] * (g.num_a * g.slots)
        return self

    def close(self) -> None:
        if self.bells is not None:
            self.bells.release()
            self.bells = None
        self.recv = None
        self.peers.clear()
        self._inbox.clear()

    # ---- handshake (the reference's server.py:181-259, as a call) ----
    def hello(self, a: int, flags: Optional[hip.HostPage], segments, geometry: Geometry) -> dict:
        """Admit A rank ``a``: the geometry must match field by field; a new epoch; the rank's
        sequence state, doorbells, unread words and half-formed jobs are reset. Returns what
        A maps: the RecvArena base, the doorbell page, the epoch and the sequence base."""
        if geometry.proto_version != self.g.proto_version:
            raise HandshakeError(f"protocol version A={geometry.proto_version} F={self.g.proto_version}")
        if geometry != self.g:
            diff = {k: (v, getattr(self.g, k)) for k, v in geometry.as_dict().items() if getattr(self.g, k) != v}
            raise HandshakeError(f"geometry mismatch (A, F): {diff}")
        if not 0 <= a < self.g.num_a:
            raise HandshakeError(f"A rank {a} outside [0, {self.g.num_a})")
        before = self.peers.get(a)
        if before is not None:
            self.stats["reconnects"] += 1
        epoch = 1 if before is None else before.epoch % MAX_EPOCH + 1
        self.peers[a] = Peer(a, flags, segments, epoch)
        slots = self.g.slots
        self._count[a * slots:(a + 1) * slots] = [self.seq_base] * slots
        self._inbox = collections.deque(m for m in self._inbox if m[0] != a)
        for s in range(slots):
            if self.bells is not None:
                self.bells.store(self.g.bell_off(a, s), self.seq_base & SEQ_MASK)
            self._forming.pop((a // self.g.group, s), None)
        return {"recv": self.recv_base, "doorbells": self.bells, "epoch": epoch, "seq_base": self.seq_base}

    # ---- discovery ----
    def announce(self, a: int, slot: int, word: int) -> None:
        """Post the doorbell word A's producer stream will write to bell(a, slot)."""
        self._inbox.append((a, slot, int(word)))

    def has_words(self) -> bool:
        """Whether posted words wait in the inbox for a poll."""
        return bool(self._inbox)

    def pending_state(self, a: int, slot: int, count: int) -> Optional[str]:
        """Where message ``count`` (its 64-bit count) that A rank ``a`` posted for ``slot``
        stands on this host: "inbox" (no poll has taken its word yet), "forming" (taken, its
        row waiting in a half-formed job for the other rows of its group) or None (handed out
        in a job, dropped by the poller's rules, or never posted)."""
        cell = a * self.g.slots + slot
        if count > self._count[cell]:
            return "inbox" if any(m[0] == a and m[1] == slot for m in self._inbox) else None
        row = self._forming.get((a // self.g.group, slot), {}).get(a % self.g.group)
        return "forming" if row is not None and row.seq == count else None

    def poll(self) -> List[Job]:
        """Every job completed by the words posted since the last call; never blocks."""
        jobs = []
        while self._inbox:
            row = self._take(*self._inbox.popleft())
            job = self._add_row(row) if row is not None else None
            if job is not None:
                jobs.append(job)
        return jobs

    def _take(self, a: int, slot: int, word: int) -> Optional[Row]:
        """Check one posted word against the rules; a Row if it starts a message to serve."""
        seq32, n_tokens, layer_id, epoch = unpack_doorbell(word)
        cell = a * self.g.slots + slot
        step = seq_ahead(seq32, self._count[cell] & SEQ_MASK)
        if step <= 0:
            return None
        self.stats["lost_messages"] += step - 1
        count = self._count[cell] = self._count[cell] + step
        peer = self.peers.get(a)
        reason = ("unknown_peer" if peer is None else
                  "stale_epoch" if epoch != peer.epoch else
                  "bad_doorbell" if not 1 <= n_tokens <= self.g.n_max else None)
        if reason is not None:
            self.stats[reason] += 1
            return None
        x_ptr = self.recv_base + self.g.region_off(a, slot)
        return Row(a=a, slot=slot, seq=count, epoch=epoch, layer_id=layer_id, n_tokens=n_tokens,
                   x_ptr=x_ptr, ids_ptr=x_ptr + self.g.ids_off, w_ptr=x_ptr + self.g.w_off)

    def _add_row(self, row: Row) -> Optional[Job]:
        group = self.g.group
        key = (row.a // group, row.slot)
        forming = self._forming.setdefault(key, {})
        forming[row.a % group] = row
        if len(forming) < group:
            return None
        del self._forming[key]
        rows = [forming[i] for i in range(group)]
        if any(r.layer_id != rows[0].layer_id for r in rows):
            self.stats["group_mismatch"] += 1
            return None
        replica = key[0]
        self.stats["jobs"] += 1
        if self._last_replica not in (None, replica):
            self.stats["replica_switches"] += 1
        self._last_replica = replica
        self.trace.append((replica, row.slot, rows[0].layer_id))
        return Job(replica=replica, slot=row.slot, layer_id=rows[0].layer_id, rows=rows,
                   t_detect_ns=time.monotonic_ns())

    # ---- the F stream: gate, answer ----
    def bell_addr(self, a: int, slot: int) -> int:
        return self.bells.addr(self.g.bell_off(a, slot))

    def gate(self, job: Job, stream: int) -> None:
        """Park ``stream`` until every row's doorbell has landed; the producer rings after its
        payload copies on the same stream, so the payload is then in the RecvArena."""
        for row in job.rows:
            hip.gate_on_doorbell(stream, self.bell_addr(row.a, row.slot), row.seq)

    def seg_view(self, row: Row):
        """A rank row.a's result segment for this F rank and the row's slot, as bf16
        [n_tokens, hidden]."""
        import torch

        g = self.g
        off = g.seg_off(self.f, row.slot) - g.flags_bytes
        seg = self.peers[row.a].segments[off : off + row.n_tokens * g.hidden * 2]
        return seg.view(torch.bfloat16).view(row.n_tokens, g.hidden)

    def seg_ptr(self, row: Row) -> int:
        """Device address of A rank row.a's result segment for this F rank and the row's slot."""
        return self.peers[row.a].segments.data_ptr() + self.g.seg_off(self.f, row.slot) - self.g.flags_bytes

    def done_addr(self, row: Row) -> int:
        """Address of the done counter whose store answers ``row``; 0 if the row's A rank
        reconnected since the row was sent (the answer is dropped: ``dropped_replies``)."""
        peer = self.peers.get(row.a)
        if peer is None or peer.epoch != row.epoch:
            self.stats["dropped_replies"] += 1
            return 0
        return peer.flags.addr(self.g.done_off(self.f, row.slot))

    def reply_job(self, job: Job, output_ptr: int, stream: int) -> None:
        """Answer every row of ``job`` in one ``afd_reply``: the row's slice of the job output
        (bf16 [sum n_tokens, hidden] at ``output_ptr``, rows in order) goes to the A rank's
        segment unless it is already there, then the A rank's done counter := the row's
        count. Rows of A ranks that reconnected since are dropped (``dropped_replies``)."""
        g = self.g
        descs = (_lib.AfdReplyDesc * len(job.rows))()
        used, offset = 0, 0
        for row in job.rows:
            nbytes = row.n_tokens * g.hidden * 2
            done = self.done_addr(row)
            if done:
                d = descs[used]
                d.src, d.dst = output_ptr + offset, self.seg_ptr(row)
                d.bytes = nbytes
                d.done = done
                d.value = row.seq
                used += 1
            offset += nbytes
        if used:
            hip.reply(descs, used, stream)

    def serve_pending(self, handler: Callable[[Job], None]) -> int:
        """Hand every job of one poll to ``handler`` (which only enqueues); returns how many."""
        jobs = self.poll()
        for job in jobs:
            handler(job)
        return len(jobs)
