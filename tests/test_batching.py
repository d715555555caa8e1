"""Host logic of the F scheduler's job batching, without a GPU: the jobs of one poll are
split into generations (the g-th message of each (replica, slot)), and each generation's jobs
are packed largest first into the first batch with room (at most batch_tokens tokens and
AFD_MAX_BATCH jobs per batch), every job exactly once, never two messages of one slot in one
batch."""

import itertools
import random
from types import SimpleNamespace

import pytest

from sgl_asap_amd import _lib
from sgl_asap_amd.runner.scheduler import FfnScheduler

_slots = itertools.count()


def job(n, layer=0, replica=None, slot=0):
    """A single-row job; by default on a (replica, slot) of its own."""
    replica = next(_slots) if replica is None else replica
    return SimpleNamespace(rows=[SimpleNamespace(n_tokens=n)], layer_id=layer, replica=replica, slot=slot)


def pack(sizes, cap):
    sched = SimpleNamespace(batch_tokens=cap)
    return [[j.rows[0].n_tokens for j in b] for b in FfnScheduler._pack(sched, [job(n) for n in sizes])]


def test_pack_largest_first_into_the_first_batch_with_room():
    assert pack([6000, 1700, 4097, 9000], 12000) == [[9000, 1700], [6000, 4097]]
    assert pack([14465, 4861, 1730, 11784], 16384) == [[14465, 1730], [11784], [4861]]
    assert pack([16384, 16384], 16384) == [[16384], [16384]]


def test_pack_holds_at_most_the_batch_job_limit():
    assert pack([1] * 20, 100) == [[1] * _lib.AFD_MAX_BATCH] * 2 + [[1] * 4]


def test_pack_random_polls_keep_every_job_once_within_capacity():
    rng = random.Random(5)
    for _ in range(300):
        cap = rng.choice([512, 4096, 16384, 32768])
        sizes = [rng.randint(1, cap) for _ in range(rng.randint(1, 24))]
        bins = pack(sizes, cap)
        assert sorted(n for b in bins for n in b) == sorted(sizes)
        for b in bins:
            assert 1 <= len(b) <= _lib.AFD_MAX_BATCH and sum(b) <= cap
            assert b == sorted(b, reverse=True)


def test_generations_split_the_messages_of_one_slot():
    a1, b1, a2, c1, a3, b2 = (job(10, replica=0, slot=0), job(20, replica=0, slot=1), job(30, replica=0, slot=0),
                              job(40, replica=1, slot=0), job(50, replica=0, slot=0), job(60, replica=0, slot=1))
    gens = FfnScheduler._generations([a1, b1, a2, c1, a3, b2])
    assert gens == [[a1, b1, c1], [a2, b2], [a3]]
    assert FfnScheduler._generations([]) == []


def test_pack_refuses_two_messages_of_one_slot():
    """Two messages of one (replica, slot) in one batched call would deadlock its F stream:
    the second's doorbell gate sits ahead of the call that answers the first."""
    sched = SimpleNamespace(batch_tokens=4096)
    with pytest.raises(ValueError, match="two messages"):
        FfnScheduler._pack(sched, [job(100, replica=3, slot=1), job(50, replica=3, slot=1)])
    # one generation at a time packs fine
    first, second = FfnScheduler._generations([job(100, replica=3, slot=1), job(50, replica=3, slot=1)])
    assert len(FfnScheduler._pack(sched, first)) == len(FfnScheduler._pack(sched, second)) == 1
