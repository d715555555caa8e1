"""Transport host logic on the CPU: doorbell and geometry known answers, the F server's
rules (cyclic sequence compare, lost messages, stale epochs, unknown peers, bad sizes,
arrival order, every posted word served, T-row jobs) against the oracle's restatement of the
reference's poller, and the stall watch (timing, release stores, poisoning), without a GPU."""

import random

import numpy as np
import pytest

from oracle import transport as OT
from sgl_asap_amd.transport import layout as L
from sgl_asap_amd.transport.channel import AttnChannel, StallWatch
from sgl_asap_amd.transport.server import FfnServer


# ---- doorbell (known answers computed from python/sgl_asap_plugin/transport/layout.py:50-53,92-102)
@pytest.mark.parametrize(
    "fields,word",
    [
        ((1, 16384, 0, 1), 0x0800400000000001),
        ((0xFFFFFFFF, 1, 60, 31), 0xF8780001FFFFFFFF),
        ((2, 8192, 3, 2), 0x1006200000000002),
        ((7, 131071, 1023, 31), 0xFFFFFFFF00000007),
    ],
)
def test_doorbell_known_answers(fields, word):
    assert L.pack_doorbell(*fields) == word
    assert L.unpack_doorbell(word) == fields
    assert OT.pack_doorbell(*fields) == word


@pytest.mark.parametrize("bad", [(1, 0, 0, 1), (1, 131072, 0, 1), (1, 1, 1024, 1), (1, 1, 0, 0), (1, 1, 0, 32)])
def test_doorbell_range_checks(bad):
    with pytest.raises(ValueError):
        L.pack_doorbell(*bad)


def test_doorbell_seq_wraps_mod_2_32():
    assert L.unpack_doorbell(L.pack_doorbell((1 << 32) + 5, 3, 0, 1))[0] == 5


def test_doorbell_roundtrip_exhaustive_fields():
    for n in (1, 2, 1000, L.MAX_TOKENS):
        for layer in (0, 1, 511, L.MAX_LAYER):
            for epoch in (1, 2, 30, L.MAX_EPOCH):
                for seq in (0, 1, 0x7FFFFFFF, 0xFFFFFFFF):
                    w = L.pack_doorbell(seq, n, layer, epoch)
                    assert L.unpack_doorbell(w) == (seq, n, layer, epoch)
                    assert w == OT.pack_doorbell(seq, n, layer, epoch)


# ---- geometry (numbers computed from layout.py:116-198 for the DSV4 rank deployment)
def test_geometry_dsv4_two_replicas_four_f():
    g = L.Geometry(num_a=2, group=1, slots=2, n_max=16384, hidden=4096, topk=8, num_f=4)
    assert g.ids_off == 134_217_728
    assert g.w_off == 134_742_016
    assert g.region_bytes == 135_266_304
    assert g.recv_bytes == 541_065_216
    assert g.flags_bytes == 2_097_152
    assert g.seg_bytes == 134_217_728
    assert g.result_bytes == 1_075_838_976
    assert g.region_off(1, 1) == 3 * 135_266_304
    assert g.bell_off(1, 0) == 128 and g.done_off(3, 1) == 7 * 64
    assert g.seg_off(1, 0) == 2_097_152 + 2 * 134_217_728
    assert g.host_bytes == 4096
    assert L.Geometry.from_dict(g.as_dict()) == g


def test_geometry_one_gpu_loop():
    g = L.Geometry(num_a=1, group=1, slots=2, n_max=8192, hidden=4096, topk=8, num_f=1)
    assert g.region_bytes == 67_633_152
    assert g.recv_bytes == 135_266_304
    assert g.result_bytes == 136_314_880


@pytest.mark.parametrize(
    "kw",
    [
        dict(num_a=0, group=1, slots=1, n_max=1, hidden=1, topk=1, num_f=1),
        dict(num_a=3, group=2, slots=1, n_max=1, hidden=1, topk=1, num_f=1),
        dict(num_a=1, group=1, slots=1, n_max=L.MAX_TOKENS + 1, hidden=1, topk=1, num_f=1),
        dict(num_a=1, group=1, slots=1.0, n_max=1, hidden=1, topk=1, num_f=1),
    ],
)
def test_geometry_rejects(kw):
    with pytest.raises(ValueError):
        L.Geometry(**kw)


def test_geometry_matches_oracle_restatement():
    for kw in (dict(num_a=3, group=3, slots=2, n_max=777, hidden=384, topk=6, num_f=2),
               dict(num_a=1, group=1, slots=1, n_max=1, hidden=256, topk=1, num_f=1)):
        g = L.Geometry(**kw)
        o = OT.geometry(**kw)
        for name in ("ids_off", "w_off", "region_bytes", "recv_bytes", "host_bytes", "flags_bytes", "seg_bytes", "result_bytes"):
            assert getattr(g, name) == o[name], name


def test_geometry_bf16_default_is_the_reference_layout():
    g = L.Geometry(num_a=1, group=1, slots=2, n_max=8192, hidden=4096, topk=8, num_f=1)
    assert g.act == "bf16" and g.xs_bytes_per_token == 0
    assert g.xs_off == g.ids_off == 8192 * 4096 * 2
    d = g.as_dict()
    del d["act"]  # a peer that predates the field
    assert L.Geometry.from_dict(d) == g


@pytest.mark.parametrize("act", ["mxfp8", "fp8_1x128"])
def test_geometry_fp8_on_the_wire(act):
    # n_max 8192, hidden 4096, topk 8: codes 32 MiB, scales 128 B/token (4096/32 UE8M0 bytes,
    # or 4096/128 fp32) = 1 MiB, ids and weights 256 KiB each
    g = L.Geometry(num_a=1, group=1, slots=2, n_max=8192, hidden=4096, topk=8, num_f=1, act=act)
    assert g.x_bytes_per_token == 4096 and g.xs_bytes_per_token == 128
    assert g.xs_off == 33_554_432
    assert g.ids_off == 34_603_008
    assert g.w_off == 34_865_152
    assert g.region_bytes == 35_127_296
    assert g.seg_bytes == 67_108_864  # results stay bf16
    assert L.Geometry.from_dict(g.as_dict()) == g
    # odd sizes: every field starts on a 256-byte boundary
    g = L.Geometry(num_a=1, group=1, slots=1, n_max=3, hidden=384, topk=3, num_f=1, act=act)
    assert g.xs_bytes_per_token == 12  # 384/32 bytes, or 3 fp32
    assert (g.xs_off, g.ids_off) == (1280, 1280 + 256)


@pytest.mark.parametrize("kw", [dict(act="fp16"), dict(act="mxfp8", hidden=200), dict(act=None)])
def test_geometry_rejects_act(kw):
    base = dict(num_a=1, group=1, slots=1, n_max=4, hidden=256, topk=1, num_f=1)
    with pytest.raises(ValueError):
        L.Geometry(**{**base, **kw})


def test_seq_ahead_cyclic():
    assert L.seq_ahead(5, 0xFFFFFFFE) == 7
    assert L.seq_ahead(0xFFFFFFFE, 5) == -7
    assert L.seq_ahead(3, 3) == 0


# ---- F server: discovery rules (the reference's server.py:262-338)
def server(num_a=2, group=1, slots=2, seq_base=0):
    g = L.Geometry(num_a=num_a, group=group, slots=slots, n_max=64, hidden=256, topk=2, num_f=1)
    s = FfnServer(0, g, memory="none", seq_base=seq_base).start()
    return s, g


def connect(s, g, a):
    return s.hello(a, None, None, g)["epoch"]


def served(jobs):
    return [(j.replica, j.slot, j.layer_id, [r.seq for r in j.rows]) for j in jobs]


def test_poll_basic_and_empty():
    s, g = server()
    e = connect(s, g, 0)
    assert s.poll() == []
    s.announce(0, 1, L.pack_doorbell(1, 10, 3, e))
    jobs = s.poll()
    assert len(jobs) == 1 and jobs[0].layer_id == 3 and jobs[0].slot == 1
    assert jobs[0].rows[0].n_tokens == 10 and jobs[0].rows[0].ids_ptr == g.region_off(0, 1) + g.ids_off
    assert jobs[0].rows[0].w_ptr == g.region_off(0, 1) + g.w_off
    assert s.poll() == []  # nothing new
    assert s.stats["jobs"] == 1 and s.trace[-1] == (0, 1, 3)


def test_two_sends_on_one_slot_before_a_poll_are_both_served_in_order():
    """The producer may post message s + 1 of a slot before the F host polled s (its stream
    then waits for the answer to s before it overwrites the region): both are served, s
    first, and nothing counts as lost."""
    s, g = server()
    e = connect(s, g, 0)
    s.announce(0, 0, L.pack_doorbell(1, 5, 0, e))
    s.announce(0, 0, L.pack_doorbell(2, 7, 1, e))
    assert s.pending_state(0, 0, 1) == s.pending_state(0, 0, 2) == "inbox"
    assert s.has_words()
    jobs = s.poll()
    assert served(jobs) == [(0, 0, 0, [1]), (0, 0, 1, [2])]
    assert s.stats["lost_messages"] == 0
    assert s.pending_state(0, 0, 1) is None and s.pending_state(0, 0, 2) is None and not s.has_words()


# ---- serving before a wait (one GPU: a wait must not be enqueued ahead of its job)
class Pump:
    """An in-process F side: serve_pending over the servers, recording the jobs."""

    def __init__(self, servers):
        self.servers, self.jobs, self.calls = servers, [], 0

    def __call__(self):
        self.calls += 1
        for sv in self.servers:
            self.jobs += sv.poll()


def test_serve_before_waiting_single_rank_rows():
    from sgl_asap_amd.transport.channel import serve_before_waiting

    s, g = server()
    e = connect(s, g, 0)
    pump = Pump([s])
    serve_before_waiting([s], 0, 0, 1, pump)  # nothing posted: nothing to do (a dropped or
    assert pump.calls == 0                     # unknown message is the stall watch's business)
    s.announce(0, 0, L.pack_doorbell(1, 5, 0, e))
    serve_before_waiting([s], 0, 0, 1, pump)
    assert pump.calls == 1 and served(pump.jobs) == [(0, 0, 0, [1])]
    serve_before_waiting([s], 0, 0, 1, pump)  # already handed out
    assert pump.calls == 1


def test_serve_before_waiting_group_of_two():
    """group = 2: the message's row may wait in a half-formed job while the word of its
    group partner is still in the inbox (a poll ran between the two sends): the wait for its
    answer serves first. With the partner's word not posted at all, no job can answer the
    message yet: the wait is refused instead of enqueued."""
    from sgl_asap_amd.transport.channel import serve_before_waiting

    s, g = server(num_a=2, group=2, slots=1)
    eps = [connect(s, g, a) for a in range(2)]
    pump = Pump([s])
    s.announce(0, 0, L.pack_doorbell(1, 4, 3, eps[0]))
    assert s.poll() == []  # rank 0's row taken, half a job
    assert s.pending_state(0, 0, 1) == "forming"
    s.announce(1, 0, L.pack_doorbell(1, 4, 3, eps[1]))  # the partner's word, not yet polled
    serve_before_waiting([s], 0, 0, 1, pump)
    assert pump.calls == 1 and served(pump.jobs) == [(0, 0, 3, [1, 1])]
    assert s.pending_state(0, 0, 1) is None and s.pending_state(1, 0, 1) is None
    # message 2 of rank 0 posted and taken, rank 1's not posted: refuse the wait
    s.announce(0, 0, L.pack_doorbell(2, 4, 4, eps[0]))
    with pytest.raises(RuntimeError, match="other A"):
        serve_before_waiting([s], 0, 0, 2, pump)
    assert pump.calls == 2 and s.pending_state(0, 0, 2) == "forming"
    # once the partner posts, the wait serves the job and goes ahead
    s.announce(1, 0, L.pack_doorbell(2, 4, 4, eps[1]))
    serve_before_waiting([s], 0, 0, 2, pump)
    assert served(pump.jobs)[-1] == (0, 0, 4, [2, 2])


def test_serve_before_waiting_ignores_later_messages():
    """A wait for message m whose job is out does not care that message m + 1 of the slot is
    still forming (its own wait is the one to check)."""
    from sgl_asap_amd.transport.channel import serve_before_waiting

    s, g = server(num_a=2, group=2, slots=1)
    eps = [connect(s, g, a) for a in range(2)]
    pump = Pump([s])
    for a in range(2):
        s.announce(a, 0, L.pack_doorbell(1, 4, 3, eps[a]))
    pump()
    s.announce(0, 0, L.pack_doorbell(2, 4, 4, eps[0]))
    pump()
    assert s.pending_state(0, 0, 2) == "forming"
    serve_before_waiting([s], 0, 0, 1, pump)  # message 1's job was handed out: no error


def test_gaps_count_as_lost_and_old_words_are_ignored():
    s, g = server()
    e = connect(s, g, 0)
    s.announce(0, 0, L.pack_doorbell(1, 5, 0, e))
    s.announce(0, 0, L.pack_doorbell(4, 5, 0, e))  # 2 and 3 were never posted
    assert served(s.poll()) == [(0, 0, 0, [1]), (0, 0, 0, [4])]
    assert s.stats["lost_messages"] == 2
    s.announce(0, 0, L.pack_doorbell(4, 5, 0, e))  # the same word again
    s.announce(0, 0, L.pack_doorbell(2, 5, 0, e))  # an older one
    assert s.poll() == [] and s.stats["lost_messages"] == 2


def test_poll_drops_stale_epoch_unknown_peer_bad_size():
    s, g = server()
    e = connect(s, g, 0)
    s.announce(0, 0, L.pack_doorbell(1, 5, 0, (e % 31) + 1))
    s.announce(1, 0, L.pack_doorbell(1, 5, 0, 1))  # rank 1 never said hello
    s.announce(0, 1, L.pack_doorbell(1, 64, 0, e))  # n == n_max is fine
    assert len(s.poll()) == 1
    assert s.stats["stale_epoch"] == 1 and s.stats["unknown_peer"] == 1
    s2, g2 = server()
    e2 = connect(s2, g2, 0)
    s2.announce(0, 0, L.pack_doorbell(1, 65, 0, e2))  # n > n_max
    assert s2.poll() == [] and s2.stats["bad_doorbell"] == 1


def test_jobs_come_out_in_arrival_order():
    s, g = server(num_a=2, slots=2)
    e = [connect(s, g, 0), connect(s, g, 1)]
    order = [(1, 1), (0, 0), (1, 0), (0, 1)]
    for a, slot in order:
        s.announce(a, slot, L.pack_doorbell(1, 4, 0, e[a]))
    assert [(j.replica, j.slot) for j in s.poll()] == order
    assert s.stats["replica_switches"] == 3


def test_sequence_field_wraps_while_counts_grow():
    base = (1 << 32) - 2
    s, g = server(seq_base=base)
    e = connect(s, g, 0)
    for m in range(1, 5):  # sequence fields 0xFFFFFFFF, 0, 1, 2
        s.announce(0, 0, L.pack_doorbell(base + m, 4, 0, e))
        jobs = s.poll()
        assert len(jobs) == 1 and jobs[0].rows[0].seq == base + m
    assert s.stats["lost_messages"] == 0


def test_group_rows_form_one_job():
    s, g = server(num_a=4, group=2, slots=1)
    eps = [connect(s, g, a) for a in range(4)]
    s.announce(1, 0, L.pack_doorbell(1, 4, 7, eps[1]))
    assert s.poll() == []  # half a job
    s.announce(0, 0, L.pack_doorbell(1, 6, 7, eps[0]))
    jobs = s.poll()
    assert len(jobs) == 1 and [r.a for r in jobs[0].rows] == [0, 1] and jobs[0].replica == 0
    s.announce(2, 0, L.pack_doorbell(1, 4, 7, eps[2]))
    s.announce(3, 0, L.pack_doorbell(1, 4, 8, eps[3]))  # the ranks of a group disagree on the layer
    assert s.poll() == [] and s.stats["group_mismatch"] == 1


def test_hello_epochs_cycle_and_reconnect_resets():
    s, g = server()
    epochs = [connect(s, g, 0) for _ in range(33)]
    assert epochs[:3] == [1, 2, 3] and epochs[30] == 31 and epochs[31] == 1
    assert s.stats["reconnects"] == 32
    e = epochs[-1]
    s.announce(0, 0, L.pack_doorbell(9, 4, 0, e))
    assert len(s.poll()) == 1
    s.announce(0, 1, L.pack_doorbell(1, 4, 0, e))  # posted, then the rank reconnects unread
    e2 = connect(s, g, 0)  # sequence state back to seq_base, unread words dropped
    assert s.poll() == []
    s.announce(0, 0, L.pack_doorbell(1, 4, 0, e2))
    assert len(s.poll()) == 1


def test_hello_rejects_geometry_mismatch():
    s, g = server()
    other = L.Geometry(num_a=2, group=1, slots=2, n_max=64, hidden=512, topk=2, num_f=1)
    with pytest.raises(L.HandshakeError):
        s.hello(0, None, None, other)
    with pytest.raises(L.HandshakeError):
        s.hello(5, None, None, g)
    fp8 = L.Geometry(**{**g.as_dict(), "act": "mxfp8"})  # same sizes, other wire format
    assert (g.proto_version, fp8.proto_version) == (L.PROTO_VERSION, L.PROTO_VERSION + 1)
    with pytest.raises(L.HandshakeError, match="protocol version"):
        s.hello(0, None, None, fp8)


def random_stream(rnd, s, g, oracle=None):
    """Random doorbell words of 3 A ranks (some never connect, some words carry a wrong
    epoch or size, some skip a sequence number)."""
    eps = {}
    for a in range(3):
        if rnd.random() < 0.8:
            eps[a] = connect(s, g, a)
            if oracle is not None:
                oracle.hello(a)
    seqs = {(a, sl): s.seq_base for a in range(3) for sl in range(2)}
    words = []
    for _ in range(40):
        a, sl = rnd.randrange(3), rnd.randrange(2)
        seqs[(a, sl)] += rnd.choice([1, 1, 1, 2])
        epoch = eps.get(a, 1) if rnd.random() < 0.9 else 17
        words.append((a, sl, L.pack_doorbell(seqs[(a, sl)], rnd.choice([1, 5, 64, 65]), rnd.randrange(4), epoch)))
    return words


def test_server_matches_oracle_poller_on_random_streams():
    """Polled after every posted word (the only order the reference's page can show, since a
    slot's doorbell cannot advance before its previous message was answered), the server
    hands out the jobs of the oracle's restatement of the reference's poller, with the same
    counts (sequence fields compared modulo 2^32)."""
    rnd = random.Random(0)
    for trial in range(20):
        s, g = server(num_a=3, slots=2, seq_base=rnd.choice([0, (1 << 32) - 5]))
        o = OT.Poller(num_a=3, group=1, slots=2, n_max=64, seq_base=s.seq_base)
        for a, sl, word in random_stream(rnd, s, g, o):
            s.announce(a, sl, word)
            o.announce(a, sl, word)
            got = [(r, sl_, lay, [q & L.SEQ_MASK for q in seqs]) for r, sl_, lay, seqs in served(s.poll())]
            assert got == o.poll(), trial
        for k, v in o.stats.items():
            assert s.stats[k] == v, (trial, k)


def test_polling_rarely_serves_the_same_jobs():
    """Every posted word stays in the inbox until a poll takes it: polling at random moments
    yields exactly the jobs (and counts) of polling after every word."""
    rnd = random.Random(1)
    for trial in range(20):
        base = rnd.choice([0, (1 << 32) - 5])
        s1, g = server(num_a=3, slots=2, seq_base=base)
        s2, _ = server(num_a=3, slots=2, seq_base=base)
        words = random_stream(random.Random(trial), s1, g)
        random_stream(random.Random(trial), s2, g)
        every, rare = [], []
        for a, sl, word in words:
            s1.announce(a, sl, word)
            every += served(s1.poll())
            s2.announce(a, sl, word)
            if rnd.random() < 0.2:
                rare += served(s2.poll())
        rare += served(s2.poll())
        assert rare == every, trial
        assert s1.stats == s2.stats


# ---- stall watch (liveness of the F side, seen from the attention rank)
class FakePage:
    """The done-counter page as the host sees it: 64-bit words at byte offsets."""

    def __init__(self, nbytes=256):
        self.words = np.zeros(nbytes // 8, dtype=np.uint64)

    def load(self, off):
        return int(self.words[off // 8])

    def store(self, off, value):
        self.words[off // 8] = np.uint64(value)


def test_stall_watch_times_unmoving_counters_and_releases_every_wait():
    page = FakePage()
    stalls = []
    w = StallWatch(page, timeout_s=1.0, on_stall=stalls.append)
    page.store(0, 3)
    page.store(64, 6)
    w.expect(0, 5, "reply #5")
    w.expect(0, 4, "send #5")  # a smaller value on the same counter adds nothing
    w.expect(64, 7, "reply on slot 1")
    assert w.scan(now=0.0) is None  # clocks start
    page.store(0, 4)  # progress on counter 0 restarts its clock
    assert w.scan(now=0.8) is None
    assert w.scan(now=1.5) == "reply on slot 1"  # counter 64 quiet since 0.0
    assert (page.load(0), page.load(64)) == (5, 7)  # every awaited value stored: waits are >=
    assert w.outstanding() == {} and w.scan(now=10.0) is None


def test_stall_watch_forgets_answered_waits():
    page = FakePage()
    w = StallWatch(page, timeout_s=0.5, on_stall=lambda what: None)
    w.expect(8, 2, "reply #2")
    assert w.scan(now=0.0) is None
    page.store(8, 9)  # answered (and later messages too)
    assert w.scan(now=5.0) is None and w.outstanding() == {}
    assert page.load(8) == 9  # nothing stored over a satisfied counter


def test_stall_poisons_the_channel():
    g = L.Geometry(num_a=1, group=1, slots=2, n_max=64, hidden=256, topk=2, num_f=1)
    ch = AttnChannel(0, g, [None], timeout_s=0.5)
    page = FakePage()
    ch.watch = StallWatch(page, 0.5, ch._stalled)
    ch.watch.expect(g.done_off(0, 1), 1, "reply to layer 3 slot 1 #1")
    ch.check()  # healthy
    assert ch.watch.scan(now=0.0) is None
    what = ch.watch.scan(now=1.0)
    ch._stalled(what)
    with pytest.raises(L.ChannelPoisoned, match="layer 3 slot 1"):
        ch.check()
    with pytest.raises(L.ChannelPoisoned):
        ch.send(3, 1, 0, 0, 0, 1, None)
    assert page.load(g.done_off(0, 1)) == 1


def test_channel_argument_checks():
    g = L.Geometry(num_a=1, group=1, slots=2, n_max=64, hidden=256, topk=2, num_f=1)
    with pytest.raises(ValueError):
        AttnChannel(1, g, [None])  # rank outside the geometry
    with pytest.raises(ValueError):
        AttnChannel(0, g, [None, None])  # one server per F rank
    with pytest.raises(ValueError):
        AttnChannel(0, g, [None], seq_base=1 << 63)
