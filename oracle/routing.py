"""Routing of one job's (token, k) pairs to this F rank's local experts (test infrastructure).

Restates the EP semantics of the expert call at
``python/sgl_asap_plugin/srt/managers/scheduler.py:410-412`` (FusedMoE with a standard
top-k output) and ``local_experts`` (``scheduler.py:206-218``): ids are global expert
ids; pairs whose id is outside ``[e_lo, e_lo + E)`` are skipped; the rest are grouped
expert by expert. The third-party kernel's order inside an expert is not pinnable, so the
build defines it: stable by flat pair index ``t * k + kk`` (``argsort(kind="stable")``).

Device layout that the HIP router produces and this oracle reproduces bit for bit:
* counts[e], offsets[e] (exclusive prefix, offsets[E] = Np);
* padded offsets: every expert segment starts on a multiple of ``block_m`` rows;
* sorted_pairs[p]: the flat pair index at padded row p, -1 on padding rows;
* pair_pos[t * k + kk]: the padded row of that pair, -1 for non-local pairs.

Pinned by brute force (a Python loop over every pair, ``route_bruteforce``) and the closed
forms above; see tests/test_oracle_routing.py.
"""

from __future__ import annotations

import numpy as np


def route(ids: np.ndarray, e_lo: int, num_local: int, block_m: int):
    """ids int32 [n, k] -> dict of counts, offsets, padded_offsets, sorted_pairs, pair_pos."""
    ids = np.asarray(ids, dtype=np.int64)
    flat = ids.reshape(-1)
    local = (flat >= e_lo) & (flat < e_lo + num_local)
    key = np.where(local, flat - e_lo, num_local)
    order = np.argsort(key, kind="stable")
    counts = np.bincount(key[local], minlength=num_local).astype(np.int32)
    offsets = np.zeros(num_local + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    padded = (counts + block_m - 1) // block_m * block_m
    poff = np.zeros(num_local + 1, dtype=np.int32)
    poff[1:] = np.cumsum(padded)
    np_pad = int(poff[-1])
    sorted_pairs = np.full(np_pad, -1, dtype=np.int32)
    pair_pos = np.full(flat.shape[0], -1, dtype=np.int32)
    n_local = int(offsets[-1])
    local_order = order[:n_local]
    expert_of = key[local_order]
    rank_in_expert = np.arange(n_local) - offsets[expert_of]
    rows = poff[expert_of] + rank_in_expert
    sorted_pairs[rows] = local_order
    pair_pos[local_order] = rows
    return {
        "counts": counts,
        "offsets": offsets,
        "padded_offsets": poff,
        "sorted_pairs": sorted_pairs,
        "pair_pos": pair_pos,
    }


def route_bruteforce(ids, e_lo: int, num_local: int, block_m: int):
    """Pure-Python restatement for tiny inputs: walk experts in order, pairs in flat order."""
    ids = [int(v) for v in np.asarray(ids).reshape(-1)]
    counts = [0] * num_local
    for v in ids:
        if e_lo <= v < e_lo + num_local:
            counts[v - e_lo] += 1
    poff = [0]
    for c in counts:
        poff.append(poff[-1] + -(-c // block_m) * block_m)
    sorted_pairs = [-1] * poff[-1]
    pair_pos = [-1] * len(ids)
    for e in range(num_local):
        row = poff[e]
        for i, v in enumerate(ids):
            if v - e_lo == e:
                sorted_pairs[row] = i
                pair_pos[i] = row
                row += 1
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    return {
        "counts": np.array(counts, dtype=np.int32),
        "offsets": np.array(offsets, dtype=np.int32),
        "padded_offsets": np.array(poff, dtype=np.int32),
        "sorted_pairs": np.array(sorted_pairs, dtype=np.int32),
        "pair_pos": np.array(pair_pos, dtype=np.int32),
    }


def local_experts(ep_rank: int, ep_size: int, num_experts: int) -> range:
    """``FfnScheduler.local_experts`` (scheduler.py:206-218): a contiguous range of
    num_experts // ep_size global ids."""
    per = num_experts // ep_size
    return range(ep_rank * per, (ep_rank + 1) * per)


def graph_buckets(max_tokens: int) -> list:
    """Powers of two below max_tokens, then max_tokens (ffn_cuda_graph_runner.py:36-39)."""
    b = [1 << i for i in range(max_tokens.bit_length()) if 1 << i < max_tokens]
    return b + [max_tokens]
