"""F side of the transport on one MI355X: the RecvArena, the doorbell page, job discovery
and replies.

Follows ``python/sgl_asap_plugin/transport/server.py``: the ``Peer`` / ``Row`` / ``Job``
records (:47-81), the handshake's epoch rule (:237, ``(old % 31) + 1``), ``poll`` with the
cyclic int32 sequence compare, lost-message count and round-robin start (:262-294), ``_row``
validation (unknown peer, stale epoch, bad n; :296-320), ``_job`` grouping of T rows
(:322-338), ``reply`` (:340-350) and the observable ``stats`` / ``trace``.

What differs on one GPU, and why:
* The reference's F host polls the doorbell page and only then launches the experts. Here
  the producer stream rings the doorbell in pinned host memory with a 64-bit stream memop,
  and the same word is posted to ``announce`` (an in-process mirror of the page), so F's host
  learns of the message without waiting for the GPU. ``run_job`` then parks F's stream on the
  real doorbell (``hip.wait64``), so the experts start when the payload has landed and no
  host thread ever waits for the GPU.
* Handshakes are calls (``hello``) instead of a TCP JSON line: A and F share a process.
"""

from __future__ import annotations

import collections
import time
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional

import numpy as np

from . import hip
from .layout import MAX_EPOCH, SEQ_MASK, Geometry, HandshakeError, unpack_doorbell


@dataclass
class Peer:
    """A connected A rank: its done-flag page, its result segments and its epoch."""

    a: int
    flags: Optional[hip.HostPage]  # A's done flags (pinned host page, FLAG_STRIDE apart)
    segments: object  # A's result segments: a device uint8 tensor at seg_off - flags_bytes
    epoch: int


@dataclass
class Row:
    """One A rank's part of a job; the pointers address this F rank's RecvArena."""

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
    """One micro-batch of one layer of one replica, ready to compute."""

    replica: int
    slot: int
    layer_id: int
    rows: List[Row]
    t_detect_ns: int


@dataclass
class _Mirror:
    words: np.ndarray = field(default_factory=lambda: np.zeros(0, dtype=np.uint64))


class FfnServer:
    """One F rank's end of the transport: ``start`` -> (``hello`` per A rank) -> ``poll`` /
    ``serve_pending`` -> ``reply`` -> ``close``.

    ``memory="none"`` skips the device and pinned allocations (host-logic tests)."""

    def __init__(self, f_rank: int, geometry: Geometry, *, device: int = 0, seq_base: int = 0,
                 memory: str = "device", trace_len: int = 4096):
        if memory not in ("device", "none"):
            raise ValueError(f"memory must be 'device' or 'none', got {memory!r}")
        self.f, self.g, self.seq_base = f_rank, geometry, seq_base & SEQ_MASK
        self.device, self.memory = device, memory
        self.stats: collections.Counter = collections.Counter()
        self.trace: collections.deque = collections.deque(maxlen=trace_len)
        self.peers: Dict[int, Peer] = {}
        self._pending: Dict[tuple, Dict[int, Row]] = {}
        self._rr = 0
        self._prev_replica = None
        self.recv = None
        self.recv_base = 0
        self.bells: Optional[hip.HostPage] = None
        self._mirror = _Mirror()
        self._last = np.zeros(0, dtype=np.uint32)

    # ---- lifetime ----
    def start(self) -> "FfnServer":
        """Allocate the RecvArena (device) and the doorbell page (pinned host); every
        doorbell starts at seq_base."""
        g = self.g
        cells = g.num_a * g.slots
        if self.memory == "device":
            import torch

            self.recv = torch.zeros(g.recv_bytes, dtype=torch.uint8, device=f"cuda:{self.device}")
            self.recv_base = self.recv.data_ptr()
            self.bells = hip.HostPage(g.host_bytes)
            for i in range(cells):
                self.bells.store(g.bell_off(i // g.slots, i % g.slots), self.seq_base)
        self._mirror.words = np.full(cells, self.seq_base, dtype=np.uint64)
        self._last = np.full(cells, self.seq_base, dtype=np.uint32)
        return self

    def close(self) -> None:
        if self.bells is not None:
            self.bells.release()
            self.bells = None
        self.recv = None
        self.peers.clear()

    # ---- handshake (server.py:181-259, as a call) ----
    def hello(self, a: int, flags: Optional[hip.HostPage], segments, geometry: Geometry) -> dict:
        """Admit A rank ``a``: check the geometry field by field, hand out a new epoch, reset
        its doorbells' last-seen sequence. Returns what A maps: recv base, doorbell page."""
        if geometry.proto_version != self.g.proto_version:
            raise HandshakeError(f"protocol version A={geometry.proto_version} F={self.g.proto_version}")
        if geometry != self.g:
            diff = {k: (v, getattr(self.g, k)) for k, v in geometry.as_dict().items() if getattr(self.g, k) != v}
            raise HandshakeError(f"geometry mismatch (A, F): {diff}")
        if not 0 <= a < self.g.num_a:
            raise HandshakeError(f"A rank {a} outside [0, {self.g.num_a})")
        old = self.peers.get(a)
        if old is not None:  # a restarted or reconnecting A rank
            self.stats["reconnects"] += 1
        epoch = (old.epoch % MAX_EPOCH) + 1 if old is not None else 1
        self.peers[a] = Peer(a, flags, segments, epoch)
        for s in range(self.g.slots):
            idx = a * self.g.slots + s
            self._mirror.words[idx] = np.uint64(self.seq_base)
            self._last[idx] = np.uint32(self.seq_base)
            if self.bells is not None:
                self.bells.store(self.g.bell_off(a, s), self.seq_base)
            self._pending.pop((a // self.g.group, s), None)  # half-assembled jobs of the old incarnation
        return {"recv": self.recv_base, "doorbells": self.bells, "epoch": epoch, "seq_base": self.seq_base}

    # ---- discovery ----
    def announce(self, a: int, s: int, word: int) -> None:
        """The doorbell word A's producer stream writes to bell(a, s); F's host reads it from
        this mirror instead of waiting for the GPU to land it."""
        self._mirror.words[a * self.g.slots + s] = np.uint64(word)

    def poll(self) -> List[Job]:
        """Jobs whose rows all arrived since the last call; never blocks (server.py:262-294)."""
        g, jobs = self.g, []
        words = self._mirror.words.copy()
        seq = (words & np.uint64(SEQ_MASK)).astype(np.uint32)
        ahead = (seq - self._last).view(np.int32)
        ready = np.flatnonzero(ahead > 0)
        if ready.size > 1:
            ready = np.concatenate([ready[ready >= self._rr], ready[ready < self._rr]])
        for idx in ready.tolist():
            a, s = divmod(idx, g.slots)
            self.stats["lost_messages"] += int(ahead[idx]) - 1
            self._last[idx] = seq[idx]
            self._rr = idx + 1
            row = self._row(a, s, int(words[idx]))
            if row is None:
                continue
            rows = self._pending.setdefault((a // g.group, s), {})
            rows[a % g.group] = row
            if len(rows) == g.group:
                job = self._job(a // g.group, s, self._pending.pop((a // g.group, s)))
                if job is not None:
                    jobs.append(job)
        return jobs

    def _row(self, a: int, s: int, word: int) -> Optional[Row]:
        seq, n_tokens, layer_id, epoch = unpack_doorbell(word)
        peer = self.peers.get(a)
        if peer is None:
            self.stats["unknown_peer"] += 1
            return None
        if epoch != peer.epoch:
            self.stats["stale_epoch"] += 1
            return None
        if not 1 <= n_tokens <= self.g.n_max:
            self.stats["bad_doorbell"] += 1
            return None
        base = self.recv_base + self.g.region_off(a, s)
        return Row(a, s, seq, epoch, layer_id, n_tokens, base, base + self.g.ids_off, base + self.g.w_off)

    def _job(self, replica: int, slot: int, rows: Dict[int, Row]) -> Optional[Job]:
        ordered = [rows[j] for j in range(self.g.group)]
        if len({r.layer_id for r in ordered}) > 1:
            self.stats["group_mismatch"] += 1
            return None
        self.stats["jobs"] += 1
        if self._prev_replica is not None and replica != self._prev_replica:
            self.stats["replica_switches"] += 1
        self._prev_replica = replica
        self.trace.append((replica, slot, ordered[0].layer_id))
        return Job(replica, slot, ordered[0].layer_id, ordered, time.monotonic_ns())

    # ---- GPU-side gate and answer ----
    def bell_addr(self, a: int, s: int) -> int:
        return self.bells.addr(self.g.bell_off(a, s))

    def wait_rows(self, job: Job, stream: int) -> None:
        """Park ``stream`` until every row's doorbell has landed (its payload copies are then
        complete: the producer rings after them, in stream order)."""
        for row in job.rows:
            hip.wait64(stream, self.bell_addr(row.a, row.slot), row.seq)

    def seg_view(self, row: Row):
        """A rank row.a's result segment for this F rank and slot, as bf16 [n_tokens, hidden]."""
        import torch

        g = self.g
        off = g.seg_off(self.f, row.slot) - g.flags_bytes
        seg = self.peers[row.a].segments[off : off + row.n_tokens * g.hidden * 2]
        return seg.view(torch.bfloat16).view(row.n_tokens, g.hidden)

    def reply(self, row: Row, src_ptr: int, nbytes: int, stream: int) -> None:
        """Enqueue: copy the partial sum into A's segment (skipped when the experts wrote it
        there), then ring A's done flag with the row's seq. Dropped if A reconnected."""
        peer, g = self.peers.get(row.a), self.g
        if peer is None or peer.epoch != row.epoch:
            self.stats["dropped_replies"] += 1
            return
        dst = self.seg_view(row).data_ptr()
        if src_ptr != dst:
            hip.copy_async(dst, src_ptr, nbytes, stream)
        hip.write64(stream, peer.flags.addr(g.done_off(self.f, row.slot)), row.seq)

    def serve_pending(self, handler: Callable[[Job], None]) -> int:
        """Hand every job found by one poll to ``handler``; returns how many."""
        jobs = self.poll()
        for job in jobs:
            handler(job)
        return len(jobs)
