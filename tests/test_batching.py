"""Host logic of the F scheduler's job batching, without a GPU: the jobs of one poll are
packed largest first into the first batch with room (at most batch_tokens tokens and
AFD_MAX_BATCH jobs per batch), every job exactly once."""

import random
from types import SimpleNamespace

from sgl_asap_amd import _lib
from sgl_asap_amd.runner.scheduler import FfnScheduler


def job(n, layer=0):
    return SimpleNamespace(rows=[SimpleNamespace(n_tokens=n)], layer_id=layer)


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
