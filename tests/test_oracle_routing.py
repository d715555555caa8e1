"""Pins the oracle's routing (CPU): the vectorised permutation against a pure-Python walk
over experts and pairs, plus its closed forms (bincount, prefix sums, block_m-aligned
segments, stability, inverse maps); and the graph-runner / EP host rules against their
known answers. Also checks that the product's host rules agree with the oracle's."""

import numpy as np
import pytest

from oracle import routing as R
from sgl_asap_amd.runner.graph_runner import graph_buckets
from sgl_asap_amd.runner.scheduler import local_experts

CASES = [
    # n, k, num_experts, e_lo, num_local, block_m
    (1, 1, 4, 0, 4, 4),
    (7, 2, 8, 0, 8, 4),
    (13, 3, 16, 4, 4, 8),
    (64, 2, 8, 0, 8, 128),
    (50, 8, 32, 8, 8, 16),
    (33, 4, 16, 12, 4, 1),
    (20, 2, 8, 100, 4, 4),  # no local experts at all
]


def _ids(n, k, num_experts, seed):
    rng = np.random.default_rng(seed)
    return np.stack([rng.choice(num_experts, k, replace=False) for _ in range(n)]).astype(np.int32).reshape(n, k)


@pytest.mark.parametrize("case", CASES)
def test_route_matches_bruteforce(case):
    n, k, ne, e_lo, nl, bm = case
    for seed in range(5):
        ids = _ids(n, k, ne, seed)
        got, want = R.route(ids, e_lo, nl, bm), R.route_bruteforce(ids, e_lo, nl, bm)
        for key in want:
            assert np.array_equal(got[key], want[key]), key


@pytest.mark.parametrize("case", CASES)
def test_route_closed_forms(case):
    n, k, ne, e_lo, nl, bm = case
    ids = _ids(n, k, ne, 11)
    r = R.route(ids, e_lo, nl, bm)
    flat = ids.reshape(-1)
    local = (flat >= e_lo) & (flat < e_lo + nl)
    assert np.array_equal(r["counts"], np.bincount(flat[local] - e_lo, minlength=nl))
    assert np.array_equal(r["offsets"], np.concatenate([[0], np.cumsum(r["counts"])]))
    seg = r["padded_offsets"]
    assert np.all(seg % bm == 0) and np.all(np.diff(seg) >= r["counts"]) and np.all(np.diff(seg) - r["counts"] < bm)
    sp, pp = r["sorted_pairs"], r["pair_pos"]
    assert np.array_equal(np.flatnonzero(pp < 0), np.flatnonzero(~local))
    assert np.array_equal(sp[pp[local]], np.flatnonzero(local))  # inverse maps
    for e in range(nl):
        rows = sp[seg[e] : seg[e] + r["counts"][e]]
        assert np.all(flat[rows] == e_lo + e)
        assert np.all(np.diff(rows) > 0)  # stable: flat pair order inside an expert
        assert np.all(sp[seg[e] + r["counts"][e] : seg[e + 1]] == -1)


def test_route_hand_example():
    """2 tokens, top-2, experts [2, 4) of 4, block 2: pairs 0:3 1:2 2:2 3:0."""
    r = R.route(np.array([[3, 2], [2, 0]], dtype=np.int32), 2, 2, 2)
    assert r["counts"].tolist() == [2, 1]
    assert r["padded_offsets"].tolist() == [0, 2, 4]
    assert r["sorted_pairs"].tolist() == [1, 2, 0, -1]
    assert r["pair_pos"].tolist() == [2, 0, 1, -1]


def test_graph_and_ep_rules_known_answers():
    assert R.graph_buckets(16384) == [1 << i for i in range(15)]
    assert R.graph_buckets(48) == [1, 2, 4, 8, 16, 32, 48]
    assert R.graph_buckets(1) == [1]
    assert R.local_experts(1, 4, 256) == range(64, 128)
    for m in (1, 2, 3, 48, 64, 100, 16384):
        assert graph_buckets(m) == R.graph_buckets(m)
    for f in range(4):
        assert local_experts(f, 4, 256) == R.local_experts(f, 4, 256)
