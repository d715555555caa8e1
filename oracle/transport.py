"""Doorbell word, arena geometry and the F poller's rules (test infrastructure).

Plain-integer restatement of ``python/sgl_asap_plugin/transport/layout.py`` and of the
poll / row / job rules of ``python/sgl_asap_plugin/transport/server.py``; written without
numpy so it shares no code path with the product's vectorised poller.

Pinned by: the four doorbell known answers and the DSV4 two-replica / four-F geometry
numbers (``tests/test_transport.py``), which were computed by hand from the bit layout
(``layout.py:40-41``) and the offset formulas (``layout.py:116-198``).
"""

from __future__ import annotations

SEQ_MASK = (1 << 32) - 1
MAX_TOKENS = (1 << 17) - 1
MAX_LAYER = (1 << 10) - 1
MAX_EPOCH = (1 << 5) - 1


def pack_doorbell(seq: int, n_tokens: int, layer_id: int, epoch: int) -> int:
    """layout.py:92-102: seq mod 2^32 | n << 32 | layer << 49 | epoch << 59."""
    assert 1 <= n_tokens <= MAX_TOKENS and 0 <= layer_id <= MAX_LAYER and 1 <= epoch <= MAX_EPOCH
    return (seq % (1 << 32)) + n_tokens * (1 << 32) + layer_id * (1 << 49) + epoch * (1 << 59)


def unpack_doorbell(word: int):
    """layout.py:105-113."""
    return word % (1 << 32), (word >> 32) % (1 << 17), (word >> 49) % (1 << 10), word >> 59


def _up(n: int, a: int) -> int:
    return -(-n // a) * a


def geometry(num_a, group, slots, n_max, hidden, topk, num_f) -> dict:
    """Every size of layout.py:116-198 as a dict (ALIGN 256, 64-byte flags and doorbells,
    the done flags in a 2 MiB page, doorbell page rounded to 4 KiB)."""
    ids_off = _up(n_max * hidden * 2, 256)
    w_off = ids_off + _up(n_max * topk * 4, 256)
    region = w_off + _up(n_max * topk * 4, 256)
    flags = _up(num_f * slots * 64, 2 << 20)
    seg = _up(n_max * hidden * 2, 256)
    return {
        "ids_off": ids_off,
        "w_off": w_off,
        "region_bytes": region,
        "recv_bytes": num_a * slots * region,
        "host_bytes": _up(num_a * slots * 64, 4096),
        "flags_bytes": flags,
        "seg_bytes": seg,
        "result_bytes": flags + num_f * slots * seg,
    }


class Poller:
    """server.py:262-338 over a plain list of doorbell words.

    ``poll`` returns ``(replica, slot, layer_id, [row seqs])`` per completed job, in the
    order the reference's poller hands them to its handler."""

    def __init__(self, num_a, group, slots, n_max, seq_base=0):
        self.num_a, self.group, self.slots, self.n_max = num_a, group, slots, n_max
        self.seq_base = seq_base % (1 << 32)
        self.words = [self.seq_base] * (num_a * slots)
        self.last = [self.seq_base] * (num_a * slots)
        self.epochs = {}
        self.pending = {}
        self.rr = 0
        self.prev_replica = None
        self.stats = {k: 0 for k in ("lost_messages", "unknown_peer", "stale_epoch", "bad_doorbell",
                                      "group_mismatch", "jobs", "replica_switches", "reconnects")}

    def hello(self, a):
        """server.py:235-250: epoch (old % 31) + 1 or 1; the rank's words and last-seen
        reset to seq_base; its half-assembled jobs dropped."""
        if a in self.epochs:
            self.stats["reconnects"] += 1
            self.epochs[a] = self.epochs[a] % MAX_EPOCH + 1
        else:
            self.epochs[a] = 1
        for s in range(self.slots):
            self.words[a * self.slots + s] = self.seq_base
            self.last[a * self.slots + s] = self.seq_base
            self.pending.pop((a // self.group, s), None)
        return self.epochs[a]

    def announce(self, a, s, word):
        self.words[a * self.slots + s] = word

    def poll(self):
        out = []
        snapshot = list(self.words)
        ready = []
        for idx, word in enumerate(snapshot):
            d = (word % (1 << 32) - self.last[idx]) % (1 << 32)
            if 0 < d < (1 << 31):  # cyclic int32 difference > 0
                ready.append((idx, d))
        if len(ready) > 1:
            ready = [r for r in ready if r[0] >= self.rr] + [r for r in ready if r[0] < self.rr]
        for idx, d in ready:
            a, s = idx // self.slots, idx % self.slots
            self.stats["lost_messages"] += d - 1
            seq, n, layer, epoch = unpack_doorbell(snapshot[idx])
            self.last[idx] = seq
            self.rr = idx + 1
            if a not in self.epochs:
                self.stats["unknown_peer"] += 1
                continue
            if epoch != self.epochs[a]:
                self.stats["stale_epoch"] += 1
                continue
            if not 1 <= n <= self.n_max:
                self.stats["bad_doorbell"] += 1
                continue
            key = (a // self.group, s)
            self.pending.setdefault(key, {})[a % self.group] = (seq, layer)
            if len(self.pending[key]) == self.group:
                rows = self.pending.pop(key)
                layers = {rows[j][1] for j in range(self.group)}
                if len(layers) > 1:
                    self.stats["group_mismatch"] += 1
                    continue
                self.stats["jobs"] += 1
                if self.prev_replica is not None and key[0] != self.prev_replica:
                    self.stats["replica_switches"] += 1
                self.prev_replica = key[0]
                out.append((key[0], s, layer, [rows[j][0] for j in range(self.group)]))
        return out
